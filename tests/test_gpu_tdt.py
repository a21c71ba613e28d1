"""GPU parity of the greedy TDT decoder (TdtDecoder::decode, src/tdt.rs:318-414;
GpuTdtDecoder::decode_async, src/tdt_gpu.rs:206-300) through the C ABI
(bark_hip_tdt_decode / bark_hip_tdt_decode_device): tokens {id, frame, dur}
equal to the transformers fixture and to the oracle, including duration-0
runs, the step guard, one-frame and empty poolers, and the device-resident
pooler of the encoder. Every case's smallest decision margin in the oracle
(best minus runner-up score) is checked to exceed the GPU's f32 rounding, so
equality is the expected outcome, not luck."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import tdt as otdt

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

GOLD = Path(__file__).resolve().parent / "golden" / "tdt_fixture.npz"
MIN_MARGIN = 1e-5  # f32 dot products of 640 terms and the LSTM state differ from f64 by ~1e-6


def make(pkg, synth, **kw):
    enc = pkg.HipEncoder.load_with(synth.SynthCheckpoint(seed=1, n_layers=1), 0, 1, decoder=synth.SynthTdt(**kw))
    return enc


@pytest.fixture(scope="module")
def base(pkg, synth):
    enc = make(pkg, synth, seed=0)
    yield enc
    enc.close()


def oracle(synth, kw, frames, pseed):
    toks, margins = otdt.Decoder(synth.SynthTdt(**kw)).decode(synth.pooler(frames, pseed), with_margins=True)
    assert margins.min() > MIN_MARGIN
    return toks


@pytest.mark.parametrize("case,frames,pseed", [("base", 300, 0), ("short", 7, 3)])
def test_tdt_vs_fixture(base, synth, case, frames, pseed):
    print(f"case tdt fixture {case}", flush=True)
    gold = np.load(GOLD, allow_pickle=False)
    np.testing.assert_array_equal(base.tdt_decode(synth.pooler(frames, pseed)), gold[f"{case}_tokens"])


@pytest.mark.parametrize("frames,pseed", [(1000, 2), (300, 1), (1, 4), (2, 5)])
def test_tdt_vs_oracle(base, synth, frames, pseed):
    print(f"case tdt oracle T={frames} seed={pseed}", flush=True)
    np.testing.assert_array_equal(base.tdt_decode(synth.pooler(frames, pseed)), oracle(synth, {"seed": 0}, frames, pseed))


def test_tdt_empty(base):
    print("case tdt empty", flush=True)
    assert base.tdt_decode(np.zeros((0, 640), np.float32)).shape == (0, 3)


def test_tdt_duration0_and_guard(pkg, synth):
    """duration-0 tokens (fixture), then a run of them that the step guard ends"""
    print("case tdt dur0 fixture", flush=True)
    gold = np.load(GOLD, allow_pickle=False)
    enc = make(pkg, synth, seed=0, dur0_bias=-0.8)
    try:
        np.testing.assert_array_equal(enc.tdt_decode(synth.pooler(300, 0)), gold["dur0_tokens"])
    finally:
        enc.close()
    print("case tdt guard", flush=True)
    enc = make(pkg, synth, seed=0, dur0_bias=-0.6)
    try:
        got = enc.tdt_decode(synth.pooler(100, 0))
        want = oracle(synth, {"seed": 0, "dur0_bias": -0.6}, 100, 0)
        assert len(want) > 1000
        np.testing.assert_array_equal(got, want)
    finally:
        enc.close()


def test_tdt_cap_too_small(pkg, base, synth):
    import ctypes

    print("case tdt cap", flush=True)
    p = np.ascontiguousarray(synth.pooler(300, 0))
    out = np.zeros((4, 3), np.uint32)
    n = ctypes.c_int32()
    rc = pkg.lib().bark_hip_tdt_decode(base._h, p.ctypes.data, 300, out.ctypes.data, 4, ctypes.byref(n))
    assert rc != 0 and n.value == 84
    assert b"token buffer too small" in pkg.lib().bark_hip_last_error()


def test_tdt_device_pooler(base, synth):
    """a pooler already in device memory (torch tensor), on torch's stream"""
    print("case tdt device", flush=True)
    p = synth.pooler(1000, 2)
    d = torch.from_numpy(p).to("cuda:0")
    s = torch.cuda.current_stream().cuda_stream
    got = base.tdt_decode_device(d.data_ptr(), 1000, s)
    np.testing.assert_array_equal(got, base.tdt_decode(p))


def test_tdt_after_encoder(pkg, synth):
    """the encoder's device-resident pooler decoded in place equals decoding
    the host copy of the same pooler (the synthetic encoder's small outputs
    leave the decision to the decoder state, so the blank bias is lowered to
    make tokens occur)"""
    print("case tdt after encoder", flush=True)
    enc = make(pkg, synth, seed=0, blank_bias=-1.0)
    try:
        mel = synth.mel(2000, 3)
        pooler, t = enc.encode_mel(mel)
        host = enc.tdt_decode(pooler)
        dm = torch.from_numpy(np.ascontiguousarray(mel)).to("cuda:0")
        dp = torch.empty((t, 640), dtype=torch.float32, device="cuda:0")
        s = torch.cuda.current_stream().cuda_stream
        n = [mel.shape[0]]
        t_out = enc.encode_mel_batch_device(dm.data_ptr(), n, n, dp.data_ptr(), dp.numel(), s)
        assert list(t_out) == [t]
        np.testing.assert_array_equal(enc.tdt_decode_device(dp.data_ptr(), t, s), host)
        assert len(host) > 0
    finally:
        enc.close()



def test_tdt_repeat_after_other_lengths(base, synth):
    """the state is reset per call: a decode after longer and shorter ones
    gives the same tokens"""
    print("case tdt repeat", flush=True)
    p = synth.pooler(300, 1)
    first = base.tdt_decode(p)
    base.tdt_decode(synth.pooler(1000, 2))
    base.tdt_decode(synth.pooler(1, 4))
    np.testing.assert_array_equal(base.tdt_decode(p), first)


def test_transcribe_wave_batch(pkg, synth):
    """waves -> tokens in one call (poolers stay on the device) equals the
    batched wave encode followed by a decode of each returned pooler"""
    print("case tdt transcribe waves", flush=True)
    enc = make(pkg, synth, seed=0, blank_bias=-1.0)
    try:
        enc.set_mel_filters()
        rng = np.random.default_rng(7)
        waves = [(0.1 * rng.standard_normal(n)).astype(np.float32) for n in (48000, 16077, 5000)]
        got = enc.transcribe_wave_batch(waves)
        poolers = enc.encode_wave_batch(waves)
        assert len(got) == len(poolers) == 3
        for g, p in zip(got, poolers):
            np.testing.assert_array_equal(g, enc.tdt_decode(p))
        assert sum(len(g) for g in got) > 0
    finally:
        enc.close()


def test_tdt_nan_inputs(pkg, synth):
    """NaN pooler rows (max(x, 0) -> 0) and NaN duration scores (no qualifying
    row: the wrapped duration ends the decode), as the oracle's reference rules"""
    print("case tdt nan", flush=True)
    import test_oracle_tdt as t

    p = synth.pooler(300, 0)
    p[40:60] = np.nan
    p[100, :7] = np.nan
    for kw, src in ((dict(seed=0), None), (dict(seed=0, blank_bias=-5.0), t._NanDurations(synth, seed=0, blank_bias=-5.0))):
        dec = src if src is not None else synth.SynthTdt(**kw)
        enc = pkg.HipEncoder.load_with(synth.SynthCheckpoint(seed=1, n_layers=1), 0, 1, decoder=dec)
        try:
            np.testing.assert_array_equal(enc.tdt_decode(p), otdt.Decoder(dec).decode(p))
        finally:
            enc.close()


def test_tdt_decode_batch(base, synth):
    """utterances decoded together (every launch advances all of them) give
    each utterance's own tokens, empty and one-frame poolers included"""
    print("case tdt batch", flush=True)
    ps = [synth.pooler(300, 1), synth.pooler(1000, 2), np.zeros((0, 640), np.float32), synth.pooler(7, 3),
          synth.pooler(1, 4)]
    got = base.tdt_decode_batch(ps)
    assert len(got) == len(ps)
    for g, p in zip(got, ps):
        np.testing.assert_array_equal(g, base.tdt_decode(p))
    np.testing.assert_array_equal(got[1], oracle(synth, {"seed": 0}, 1000, 2))


def test_transcribe_vs_cpu_oracles(pkg, synth):
    """wave -> tokens on the GPU equals the CPU oracles chained (numpy log-mel,
    the C encoder restatement, the numpy TDT decode) on a 3 s wave; the
    oracle's smallest decision margin is checked to exceed the encoder's
    f16 rounding, so equality is expected"""
    import importlib

    import oracle
    from oracle import mel as omel

    print("case tdt transcribe vs oracles", flush=True)
    src = synth.SynthCheckpoint(seed=3, n_layers=2, style="rich", lowbit=True)
    dec = synth.SynthTdt(seed=0, blank_bias=1.5)
    enc = pkg.HipEncoder.load_with(src, 0, 2, decoder=dec)
    try:
        filters = importlib.import_module("bark3_wgpu_amd.mel").slaney_mel_filters()
        enc.set_mel_filters(filters)
        rng = np.random.default_rng(11)
        n = 48000
        t = np.arange(n) / 16000.0
        wave = (0.3 * np.sin(2 * np.pi * (220 + 300 * t) * t) + 0.05 * rng.standard_normal(n)).astype(np.float32)
        got = enc.transcribe_wave_batch([wave])[0]
    finally:
        enc.close()
    feats, frames, valid = omel.features(wave, filters)
    sub = oracle.subsample(src, feats, valid)
    T = pkg.conv_len(pkg.conv_len(pkg.conv_len(frames)))
    pooler = oracle.Encoder(src, 2).encode(sub, T)
    want, margins = otdt.Decoder(dec).decode(pooler, with_margins=True)
    assert margins.min() > 2e-3, f"oracle decision margin {margins.min():.2e} too small for this check"
    assert len(want) > 0
    np.testing.assert_array_equal(got, want)


def test_tdt_error_paths(pkg, synth):
    """no decoder tensors, no mel filters, bad lengths: clear errors, no decode"""
    print("case tdt errors", flush=True)
    enc = pkg.HipEncoder.load_with(synth.SynthCheckpoint(seed=1, n_layers=1), 0, 1)
    try:
        with pytest.raises(pkg.HipError, match="no TDT decoder tensors"):
            enc.tdt_decode(synth.pooler(5, 0))
    finally:
        enc.close()
    enc = make(pkg, synth, seed=0)
    try:
        with pytest.raises(pkg.HipError, match="set_mel_filters"):
            enc.transcribe_wave_batch([np.zeros(1600, np.float32)])
        import ctypes

        out = np.zeros((4, 3), np.uint32)
        n = ctypes.c_int32()
        p = np.ascontiguousarray(synth.pooler(2, 0))
        assert pkg.lib().bark_hip_tdt_decode(enc._h, p.ctypes.data, -1, out.ctypes.data, 4, ctypes.byref(n)) != 0
        assert b"t_len out of range" in pkg.lib().bark_hip_last_error()
        # the handle still decodes after the errors
        np.testing.assert_array_equal(enc.tdt_decode(synth.pooler(7, 3)), oracle(synth, {"seed": 0}, 7, 3))
    finally:
        enc.close()
