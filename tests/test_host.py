"""Host-side logic that needs no GPU: tensor naming, synthetic checkpoints,
the 4-bit adapters and the bench contract."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]


def test_tensor_names_match_reference_loader(pkg, oracle):
    names = pkg.tensor_names(24)
    assert len(names) == len(set(names)) == 10 + 2 + 24 * 28 + 2
    assert "encoder.layers.23.conv.depthwise_conv.weight" in names
    per_layer = [n.split(".", 3)[3] for n in names if n.startswith("encoder.layers.0.")]
    assert sorted(per_layer) == sorted(oracle.LAYER_TENSORS)


def test_conv_len_chain(pkg, oracle):
    for f in (1, 2, 3, 61, 1500, 17656, 120000):
        t = pkg.conv_len(pkg.conv_len(pkg.conv_len(f)))
        assert t == oracle.conv_len(oracle.conv_len(oracle.conv_len(f)))
    assert pkg.conv_len(pkg.conv_len(pkg.conv_len(1500))) == 188
    assert pkg.conv_len(pkg.conv_len(pkg.conv_len(17656))) == 2207
    assert pkg.conv_len(pkg.conv_len(pkg.conv_len(120000))) == 15000


def test_synth_is_deterministic_and_bf16(synth):
    a = synth.SynthCheckpoint(seed=9, n_layers=2)
    b = synth.SynthCheckpoint(seed=9, n_layers=2)
    w = a.read("encoder.layers.1.feed_forward1.linear1.weight")
    assert w.shape == (4096, 1024)
    assert np.array_equal(w, b.read("encoder.layers.1.feed_forward1.linear1.weight"))
    assert np.all((w.view(np.uint32) & 0xFFFF) == 0)  # bf16 values
    assert abs(float(w.std()) - 0.02) < 1e-3


def test_synth_lowbit_formats_dequantize_consistently(synth, oracle):
    for fmt in ("lut16", "levels"):
        src = synth.SynthCheckpoint(seed=2, n_layers=1, lowbit=True, lowbit_format=fmt, k_lev=3)
        name = "encoder.layers.0.self_attn.o_proj.weight"
        t = src.read_lowbit(name)
        deq = src.read(name)
        if fmt == "lut16":
            want = oracle.lut4_expand(t.codes, t.lut16, t.rows, t.cols)
            assert set(np.unique(t.codes & 15)) == set(range(16))
        else:
            want = oracle.lowbit_expand(t.codes, t.levels, t.k, t.rows, t.cols)
            assert int(((t.codes >> 0) & 15).max()) <= 2 * t.k
        assert np.array_equal(deq.view(np.uint32), want.view(np.uint32))
    assert synth.SynthCheckpoint(lowbit=True).read_lowbit("encoder_projector.weight") is None


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr
