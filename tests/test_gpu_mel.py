"""GPU parity of the log-mel front end (MelFrontend::compute, src/mel.rs:41-140)
through the C ABI (bark_hip_set_mel_filters / bark_hip_mel / bark_hip_mel_device)
against the oracle and the torch.stft fixture."""
from __future__ import annotations

import importlib
from pathlib import Path

import numpy as np
import pytest

from oracle import mel as omel

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

GOLD = Path(__file__).resolve().parent / "golden" / "mel_fixture.npz"
TOL = 1e-3  # f32 radix-2 FFT and f64 statistics vs the f64 pipelines


@pytest.fixture(scope="module")
def fe(pkg):
    enc = pkg.HipEncoder(0, 1)
    enc.set_mel_filters(importlib.import_module("bark3_wgpu_amd.mel").slaney_mel_filters())
    yield enc
    enc.close()


@pytest.fixture(scope="module")
def filters(pkg):
    return importlib.import_module("bark3_wgpu_amd.mel").slaney_mel_filters()


@pytest.mark.parametrize("k", ["a", "b", "c"])
def test_mel_vs_fixture_and_oracle(fe, filters, k):
    print(f"case mel fixture {k}", flush=True)
    gold = np.load(GOLD, allow_pickle=False)
    w = gold[f"wave_{k}"]
    got, nf, nv = fe.mel(w)
    assert (nf, nv) == (int(gold[f"frames_{k}"]), int(gold[f"valid_{k}"]))
    assert np.abs(got - gold[f"feat_{k}"]).max() <= TOL
    want, _, _ = omel.features(w, filters)
    assert np.abs(got - want).max() <= TOL
    assert not got[nv:].any()


@pytest.mark.parametrize("n", [1, 159, 160, 161, 48000 + 77])
def test_mel_lengths(fe, filters, n):
    print(f"case mel length {n}", flush=True)
    rng = np.random.default_rng(n)
    w = (0.1 * rng.standard_normal(n)).astype(np.float32)
    got, nf, nv = fe.mel(w)
    want, wf, wv = omel.features(w, filters)
    assert (nf, nv) == (wf, wv) == (1 + n // 160, n // 160)
    assert np.abs(got - want).max() <= TOL


def test_mel_device_long_utterance(fe, filters):
    """176.56 s (the encoder benchmark's 17656 frames) on device buffers."""
    n = 160 * 17655 + 100
    print(f"case mel device n={n}", flush=True)
    rng = np.random.default_rng(7)
    t = np.arange(n) / 16000.0
    w = (0.2 * np.sin(2 * np.pi * (300 + 40 * t) * t) + 0.02 * rng.standard_normal(n)).astype(np.float32)
    d_w = torch.from_numpy(w).cuda()
    nf = 1 + n // 160
    d_out = torch.empty((nf, 128), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    frames, valid = fe.mel_device(d_w.data_ptr(), n, d_out.data_ptr(), d_out.numel(), stream)
    torch.cuda.synchronize()
    assert (frames, valid) == (nf, n // 160) == (17656, 17655)
    want, _, _ = omel.features(w, filters)
    err = np.abs(d_out.cpu().numpy() - want)
    # the f64 FFT's power rounded to f32 and f32 mel sums: f32 rounding (an f32
    # FFT such as the reference's reaches ~1.4e-4 here against this f64 oracle)
    assert err.max() <= TOL
    assert np.quantile(err, 0.999) <= 1e-4


def test_encode_wave_batch_equals_individual(pkg, synth, filters):
    """bark_hip_encode_wave_batch = each wave's own mel + encode_mel, exactly
    (chunked transcription as one batched call)."""
    rng = np.random.default_rng(11)
    lens = [14400 + 37, 36800 + 5, 24000]
    print(f"case wave batch lens={lens}", flush=True)
    waves = [(0.1 * rng.standard_normal(n)).astype(np.float32) for n in lens]
    src = synth.SynthCheckpoint(seed=11, n_layers=2, style="rich", lowbit=True)
    with pkg.HipEncoder.load_with(src, n_layers=2) as enc:
        enc.set_mel_filters(filters)
        batch = enc.encode_wave_batch(waves)
        singles = []
        for w in waves:
            feats, nf, nv = enc.mel(w)
            singles.append(enc.encode_mel(feats, nv)[0])
    for b, s in zip(batch, singles):
        assert b.shape == s.shape
        assert np.array_equal(b, s)
