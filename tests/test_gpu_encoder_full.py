"""Full-encoder GPU parity: every block's pre-norm residual and the pooler
against the CPU oracle, batched packing, length masks, long streams and the
reference's own low-bit format. Tolerance (BASELINE): relative max-abs error
<= 1e-2 per block; the measured per-layer table is printed."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_max_abs

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _per_layer(enc, orc, sub, t, n_layers, layers):
    want_pool, want_dumps = orc.encode_dump(sub, t)
    errs = []
    for l in layers:
        got = enc.encode(sub, t, dump_layer=l)
        errs.append((l, rel_max_abs(got.block, want_dumps[l])))
    pool = enc.encode(sub, t).pooler
    return errs, rel_max_abs(pool, want_pool)


def test_config2_full_encoder_t188(pkg, synth, oracle):
    """24 blocks, bf16 weights, log-mel [1500,128] -> T=188, via
    the conv front end; per-layer errors from encode() dumps."""
    print("case config2 t=188", flush=True)
    src = synth.SynthCheckpoint(seed=21, n_layers=24, style="rich")
    mel = synth.mel(1500, seed=21)
    with pkg.HipEncoder.load_with(src, n_layers=24) as enc:
        pooler, t = enc.encode_mel(mel)
        assert t == 188
        orc = oracle.Encoder(src, 24)
        sub = oracle.subsample(src, mel)
        errs, e_pool_sub = _per_layer(enc, orc, sub, t, 24, range(24))
    want = orc.encode(sub, t)
    e_pool = rel_max_abs(pooler, want)
    print("  per-layer rel max-abs:", " ".join(f"{l}:{e:.1e}" for l, e in errs))
    print(f"  pooler (mel path) {e_pool:.2e}, pooler (sub path) {e_pool_sub:.2e}")
    assert max(e for _, e in errs) <= TOL
    assert e_pool <= TOL and e_pool_sub <= TOL


def test_config3_lowbit_t2207(pkg, synth, oracle):
    """24 blocks with 4-bit linears, log-mel [17656,128] -> T=2207."""
    print("case config3 t=2207", flush=True)
    src = synth.SynthCheckpoint(seed=31, n_layers=24, style="rich", lowbit=True)
    mel = synth.mel(17656, seed=31)
    with pkg.HipEncoder.load_with(src, n_layers=24) as enc:
        pooler, t = enc.encode_mel(mel)
        assert t == 2207
        orc = oracle.Encoder(src, 24)
        sub = oracle.subsample(src, mel)
        want_pool, want_dumps = orc.encode_dump(sub, t)
        errs = [(l, rel_max_abs(enc.encode(sub, t, dump_layer=l).block, want_dumps[l])) for l in range(24)]
    e_pool = rel_max_abs(pooler, want_pool)
    print("  per-layer rel max-abs (pre-norm residual of each block vs the oracle):")
    for l, e in errs:
        print(f"    layer {l:2d}  {e:.2e}")
    print(f"    pooler    {e_pool:.2e}")
    assert max(e for _, e in errs) <= TOL and e_pool <= TOL


def test_config4_batch_16_utterances(pkg, synth, oracle):
    """configs[4] at its real workload: 16 utterances of U(5, 60) s (seeded)
    through the 24-block 4-bit encoder as one packed batch. Every utterance
    equals its own batch-1 encode_mel bit for bit (the reference runs the
    chunks one after another, src/inference.rs:311-326), and the shortest and
    the longest match the oracle per layer."""
    rng = np.random.default_rng(4)
    secs = rng.uniform(5.0, 60.0, size=16)
    frames = [int(s * 100) for s in secs]
    ts = [pkg.conv_len(pkg.conv_len(pkg.conv_len(f))) for f in frames]
    print(f"case config4 batch of 16: frames={frames} T={ts}", flush=True)
    src = synth.SynthCheckpoint(seed=44, n_layers=24, style="rich", lowbit=True)
    mels = [synth.mel(f, seed=100 + i) for i, f in enumerate(frames)]
    with pkg.HipEncoder.load_with(src, n_layers=24) as enc:
        batch = enc.encode_mel_batch(mels)
        singles = [enc.encode_mel(m)[0] for m in mels]
        for i, (b, s1) in enumerate(zip(batch, singles)):
            assert b.shape == (ts[i], 640) and b.shape == s1.shape
            assert np.array_equal(b, s1), f"utterance {i} (T={ts[i]}) differs from its own encode"
        print("  16 of 16 batch results bit-identical to their batch-1 encodes", flush=True)
        orc = oracle.Encoder(src, 24)
        for i in (int(np.argmin(frames)), int(np.argmax(frames))):
            sub = oracle.subsample(src, mels[i])
            t = ts[i]
            want_pool, want_dumps = orc.encode_dump(sub, t)
            errs = [rel_max_abs(enc.encode(sub, t, dump_layer=l).block, want_dumps[l]) for l in range(24)]
            e_pool = rel_max_abs(batch[i], want_pool)
            print(f"  utterance {i} T={t}: per-layer max {max(errs):.2e} (layer {int(np.argmax(errs))}), "
                  f"batched pooler {e_pool:.2e}", flush=True)
            assert max(errs) <= TOL and e_pool <= TOL


def test_two_streams_back_to_back(pkg, synth):
    """Device-form calls on one handle from two streams, queued back to back
    without a host synchronisation between them: the second call waits for the
    first on the device (they share the handle's workspace), so both results
    equal single-stream runs."""
    import torch

    src = synth.SynthCheckpoint(seed=45, n_layers=2, style="rich", lowbit=True)
    fa, fb = 2400, 1300
    ma, mb = synth.mel(fa, seed=1), synth.mel(fb, seed=2)
    ta = pkg.conv_len(pkg.conv_len(pkg.conv_len(fa)))
    tb = pkg.conv_len(pkg.conv_len(pkg.conv_len(fb)))
    print(f"case two streams T={ta},{tb}", flush=True)
    with pkg.HipEncoder.load_with(src, n_layers=2) as enc:
        want_a, _ = enc.encode_mel(ma)
        want_b, _ = enc.encode_mel(mb)
        da, db = torch.from_numpy(ma).cuda(), torch.from_numpy(mb).cuda()
        pa = torch.full((ta, 640), float("nan"), device="cuda")
        pb = torch.full((tb, 640), float("nan"), device="cuda")
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        torch.cuda.synchronize()
        for _ in range(3):
            enc.encode_mel_batch_device(da.data_ptr(), [fa], [fa], pa.data_ptr(), pa.numel(), s1.cuda_stream)
            enc.encode_mel_batch_device(db.data_ptr(), [fb], [fb], pb.data_ptr(), pb.numel(), s2.cuda_stream)
        torch.cuda.synchronize()
        got_a, got_b = pa.cpu().numpy(), pb.cpu().numpy()
    assert np.array_equal(got_a, want_a) and np.array_equal(got_b, want_b)


def test_graph_replays_equal_eager(pkg, synth):
    """A repeated packing replays a captured HIP graph of the encode (the first
    call runs eagerly, the second captures). Every replay, with eager work and
    synchronisations in between (another packing, torch kernels, the isolated
    linear), equals the eager result bit for bit."""
    import torch

    src = synth.SynthCheckpoint(seed=46, n_layers=2, style="rich", lowbit=True)
    fa, fb = 1500, 700
    ma, mb = synth.mel(fa, seed=3), synth.mel(fb, seed=4)
    ta = pkg.conv_len(pkg.conv_len(pkg.conv_len(fa)))
    tb = pkg.conv_len(pkg.conv_len(pkg.conv_len(fb)))
    print(f"case graph replays T={ta},{tb}", flush=True)
    with pkg.HipEncoder.load_with(src, n_layers=2) as enc:
        da, db = torch.from_numpy(ma).cuda(), torch.from_numpy(mb).cuda()
        pa = torch.empty((ta, 640), device="cuda")
        pb = torch.empty((tb, 640), device="cuda")
        sp = torch.cuda.current_stream().cuda_stream

        def run_a():
            pa.fill_(float("nan"))
            enc.encode_mel_batch_device(da.data_ptr(), [fa], [fa], pa.data_ptr(), pa.numel(), sp)
            torch.cuda.synchronize()
            return pa.cpu().numpy().copy()

        def run_b():
            pb.fill_(float("nan"))
            enc.encode_mel_batch_device(db.data_ptr(), [fb], [fb], pb.data_ptr(), pb.numel(), sp)
            torch.cuda.synchronize()
            return pb.cpu().numpy().copy()

        want_a = run_a()  # eager
        want_b, _ = enc.encode_mel(mb)
        A = torch.randn((64, 1024), device="cuda").to(torch.bfloat16)
        codes = torch.randint(0, 256, (1024, 512), device="cuda", dtype=torch.uint8)
        lut = torch.sort(torch.randn((1024, 16), device="cuda") * 0.02, dim=1).values.half()
        C = torch.empty((64, 1024), device="cuda", dtype=torch.bfloat16)
        for i in range(6):  # capture on the first repeat, replays after
            assert np.array_equal(run_a(), want_a), f"replay {i} differs from the eager encode"
            x = torch.randn(4096, device="cuda").cumsum(0)  # eager torch work between replays
            pkg.lowbit_linear(A.data_ptr(), 1, codes.data_ptr(), lut.data_ptr(), C.data_ptr(), 2, 64, 1024, 1024, sp)
            torch.cuda.synchronize()
            assert bool(torch.isfinite(x).all())
        # alternating packings: each call still equals its eager result
        for i in range(4):
            assert np.array_equal(run_b(), want_b), f"packing B, round {i}"
            assert np.array_equal(run_a(), want_a), f"packing A after B, round {i}"


def test_batch_equals_individual(pkg, synth):
    """configs[4] semantics: each utterance of a packed batch equals its own
    batch-1 run (identical per-row arithmetic, so the match is exact)."""
    rng = np.random.default_rng(41)
    frames = [int(x) for x in rng.integers(500, 3000, size=5)]
    print(f"case batch frames={frames}", flush=True)
    src = synth.SynthCheckpoint(seed=41, n_layers=2, style="rich", lowbit=True)
    mels = [synth.mel(f, seed=i) for i, f in enumerate(frames)]
    with pkg.HipEncoder.load_with(src, n_layers=2) as enc:
        batch = enc.encode_mel_batch(mels)
        singles = [enc.encode_mel(m)[0] for m in mels]
    for b, s in zip(batch, singles):
        assert b.shape == s.shape
        assert np.array_equal(b, s)


def test_short_inputs_equal_their_batched_rows(pkg, synth):
    """Inputs of at most 256 frames run the short-input GEMM tiles (weight
    fragments made once per workgroup, 4-bit and f16 weights alike); packed
    with a long one they run the long-input tiles. The per-element MFMA order
    is the same, so the results are identical bit for bit."""
    frames = [1500, 800, 300, 4000]  # T = 188, 100, 38, 500
    for lowbit in (True, False):
        print(f"case short vs batched frames={frames} lowbit={lowbit}", flush=True)
        src = synth.SynthCheckpoint(seed=43, n_layers=2, style="rich", lowbit=lowbit)
        mels = [synth.mel(f, seed=10 + i) for i, f in enumerate(frames)]
        with pkg.HipEncoder.load_with(src, n_layers=2) as enc:
            batch = enc.encode_mel_batch(mels)
            singles = [enc.encode_mel(m)[0] for m in mels]
        for b, s in zip(batch, singles):
            assert b.shape == s.shape
            assert np.array_equal(b, s)


def test_relk_table_growth_keeps_results(pkg, synth):
    """The relative keys of every layer are computed once per position-table
    length and kept: a longer input grows the table and recomputes them (and
    retires graphs captured before), shorter inputs read a sub-range. Each
    encode equals the same encode on a fresh handle, bit for bit, through
    graph replays before and after the growth."""
    src = synth.SynthCheckpoint(seed=47, n_layers=2, style="rich", lowbit=True)
    fa, fb = 1500, 6000  # T = 188, then T = 750 (table 256 -> 750 rows)
    ma, mb = synth.mel(fa, seed=5), synth.mel(fb, seed=6)
    print(f"case relK table growth frames={fa},{fb}", flush=True)
    with pkg.HipEncoder.load_with(src, n_layers=2) as fresh:
        want_a = fresh.encode_mel(ma)[0]
    with pkg.HipEncoder.load_with(src, n_layers=2) as fresh:
        want_b = fresh.encode_mel(mb)[0]
    with pkg.HipEncoder.load_with(src, n_layers=2) as enc:
        for i in range(3):  # eager, capture, replay
            assert np.array_equal(enc.encode_mel(ma)[0], want_a), f"short input, call {i}"
        assert np.array_equal(enc.encode_mel(mb)[0], want_b), "longer input (table grows)"
        for i in range(4):
            assert np.array_equal(enc.encode_mel(ma)[0], want_a), f"short input after growth, call {i}"
        assert np.array_equal(enc.encode_mel(mb)[0], want_b), "longer input again"


def test_n_valid_masks_front_end(pkg, synth, oracle):
    """n_valid < n_frames zeroes the masked frames after each strided conv
    (src/sub.rs:259-273)."""
    src = synth.SynthCheckpoint(seed=51, n_layers=1, style="rich")
    mel = synth.mel(800, seed=51)
    with pkg.HipEncoder.load_with(src, n_layers=1) as enc:
        got, t = enc.encode_mel(mel, n_valid=523)
    sub = oracle.subsample(src, mel, n_valid=523)
    want = oracle.Encoder(src, 1).encode(sub, t)
    err = rel_max_abs(got, want)
    print(f"case n_valid=523 of 800: pooler err {err:.2e}")
    assert err <= TOL


@pytest.mark.parametrize("t", [4096, 15000])
def test_long_stream_one_block(pkg, synth, oracle, t):
    """Past the reference's 4096-frame fused-softmax limit and the 20-minute
    stream of configs[4] (T=15000): flash attention keeps O(T) memory."""
    print(f"case long stream t={t}", flush=True)
    src = synth.SynthCheckpoint(seed=61, n_layers=1, style="rich", lowbit=True)
    sub = np.random.default_rng([t, 61]).standard_normal((t, 4096), dtype=np.float32)
    with pkg.HipEncoder.load_with(src, n_layers=1, front_end=False) as enc:
        got = enc.encode(sub, t, dump_layer=0)
    want_pool, want_dumps = oracle.Encoder(src, 1).encode_dump(sub, t)
    e_blk, e_pool = rel_max_abs(got.block, want_dumps[0]), rel_max_abs(got.pooler, want_pool)
    print(f"  block err {e_blk:.2e} pooler err {e_pool:.2e}")
    assert e_blk <= TOL and e_pool <= TOL


@pytest.mark.parametrize("t", [200, 1500])
def test_reference_lowbit_format_equals_f16(pkg, synth, t):
    """The reference's LowBitTensor path (codes in 0..2k, k levels per row)
    gives bit-identical results to f16 weights holding the expanded values —
    the invariant of the reference's `lbtest` (src/diagnostics/gemm.rs:538-652).
    T = 200 runs the short-input strip tiles, T = 1500 the eight-wave tiles
    (qkv, FFN down) and the four-wave ones."""
    low = synth.SynthCheckpoint(seed=71, n_layers=1, style="rich", lowbit=True, lowbit_format="levels", k_lev=3)

    class Expanded:
        def read(self, name):
            v = low.read(name)
            return v.astype(np.float16) if low.read_lowbit(name) is not None else v

        def read_lowbit(self, name):
            return None

    print(f"case lbtest invariant T={t}", flush=True)
    sub = np.random.default_rng(71).standard_normal((t, 4096), dtype=np.float32)
    with pkg.HipEncoder.load_with(low, n_layers=1, front_end=False) as a:
        ya = a.encode(sub, t, dump_layer=0)
    with pkg.HipEncoder.load_with(Expanded(), n_layers=1, front_end=False) as b:
        yb = b.encode(sub, t, dump_layer=0)
    assert np.array_equal(ya.pooler, yb.pooler) and np.array_equal(ya.block, yb.block)
