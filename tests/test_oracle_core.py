"""Pins of the CPU oracle's primitives against checks independent of its own
formulas: numpy's IEEE casts, closed forms, brute force and the reference's own
unit-test shapes and known-answer generators."""
from __future__ import annotations

import math

import numpy as np
import pytest


# ---------------------------------------------------------------- conversions
def test_f32_to_f16_matches_numpy_rne(oracle):
    """src/raw.rs:130-133 (half::f16::from_f32, round-to-nearest-even) checked
    against numpy's float16 cast on random values and every edge class."""
    rng = np.random.default_rng(0)
    edge = np.array(
        [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf, 6.1035156e-05,
         5.9604645e-08, 2.9802322e-08, 2.98023259e-08, 1e-10, 1.0009765625, 1.00048828125, 1.00146484375,
         2049.0, 2051.0, -2049.0, 3.0517578e-05],
        np.float32,
    )
    vals = np.concatenate([edge, rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 100000)])
    vals = vals.astype(np.float32)
    got = oracle.f32_to_f16_bits(vals)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    # widening back is exact
    assert np.array_equal(oracle.round_f16(vals), vals.astype(np.float16).astype(np.float32))


def test_f16_ties_round_to_even(oracle):
    # 1 + 2^-11 is halfway between 1 and 1 + 2^-10: ties go to the even mantissa (1.0)
    assert oracle.lib().bo_f32_to_f16(1.0 + 2.0**-11) == 0x3C00
    assert oracle.lib().bo_f32_to_f16(1.0 + 3 * 2.0**-11) == 0x3C02


def test_bf16_widen_is_a_shift(oracle):
    """src/raw.rs:118-120: bf16 bits b -> f32 bits b << 16."""
    for b in (0x0000, 0x8000, 0x3F80, 0xBF80, 0x7F80, 0x4049, 0x0001):
        want = np.array([b << 16], np.uint32).view(np.float32)[0]
        got = oracle.lib().bo_bf16_to_f32(b)
        assert np.float32(got).view(np.uint32) == want.view(np.uint32)


# ------------------------------------------------------------------- low-bit
def test_expand_table_closed_form(oracle):
    """src/bark.rs:597-611: 0 -> 0, 1..k -> +lev, k+1..2k -> -lev, above 2k a
    missing level reads 0 and is negated."""
    lev16 = np.array([0.25, 0.5, 0.75, 0.0], np.float16).view(np.uint16)
    for k in (1, 2, 3):
        lv = lev16.view(np.float16).astype(np.float32)
        for c in range(16):
            got = oracle.expand(c, k, lev16)
            if c == 0:
                want = 0.0
            elif c <= k:
                want = lv[c - 1]
            elif c <= 2 * k:
                want = -lv[c - k - 1]
            else:
                want = -0.0
            assert got == want and math.copysign(1, got) == math.copysign(1, want), (k, c)


def test_lbtest_generator_layout(oracle):
    """The reference's low-bit known-answer pattern (src/diagnostics/gemm.rs:
    538-652): levels[row] = [0.02*(row%7+1), 0.05*(row%5+1)], codes[i] =
    (i*13 + i/k) % 5 with k = 1024 columns. The u32 nibble layout expands to the
    same values as two-codes-per-byte (byte-identical on little endian)."""
    n, kk, k_lev = 128, 1024, 2
    lev = np.zeros((n, 4), np.float16)
    rows = np.arange(n)
    lev[:, 0] = 0.02 * (rows % 7 + 1)
    lev[:, 1] = 0.05 * (rows % 5 + 1)
    i = np.arange(n * kk, dtype=np.int64)
    codes = ((i * 13 + i // kk) % 5).astype(np.uint32).reshape(n, kk)
    words = np.zeros((n, kk // 8), np.uint32)
    for e in range(8):
        words |= codes[:, e::8] << np.uint32(4 * e)
    a = oracle.lowbit_expand(words, lev.view(np.uint16), k_lev, n, kk)
    # closed form
    lv = lev.astype(np.float32)
    want = np.zeros((n, kk), np.float32)
    want[codes == 1] = np.broadcast_to(lv[:, [0]], (n, kk))[codes == 1]
    want[codes == 2] = np.broadcast_to(lv[:, [1]], (n, kk))[codes == 2]
    want[codes == 3] = -np.broadcast_to(lv[:, [0]], (n, kk))[codes == 3]
    want[codes == 4] = -np.broadcast_to(lv[:, [1]], (n, kk))[codes == 4]
    assert np.array_equal(a, want)
    # the same bytes read as the generic two-per-byte layout with a 16-entry table
    lut = np.zeros((n, 16), np.float16)
    for c in range(16):
        lut[:, c] = [oracle.expand(c, k_lev, lev[r].view(np.uint16)) for r in range(n)]
    b = oracle.lut4_expand(words.view(np.uint8), lut.view(np.uint16), n, kk)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---------------------------------------------------------------------- GEMM
def _naive(a, w):
    return a.astype(np.float64) @ w.astype(np.float64).T


@pytest.mark.parametrize("m,n,k", [(1, 16, 5), (7, 40, 33), (13, 128, 64), (191, 64, 17)])
def test_gemm_matches_naive_for_odd_shapes(oracle, m, n, k):
    """src/cpu/gemm.rs:787-802 (same inputs, same 1e-4 bound)."""
    a = ((np.arange(m * k) % 17) * 0.01 - 0.05).astype(np.float32).reshape(m, k)
    w = ((np.arange(n * k) % 13) * 0.02 - 0.1).astype(np.float32).reshape(n, k)
    c = oracle.gemm(a, oracle.PackW(w))
    assert np.max(np.abs(c - _naive(a, w))) < 1e-4


@pytest.mark.parametrize("m,n,k", [(6, 16, 16), (13, 40, 33), (24, 128, 64), (7, 96, 40)])
def test_half_pack_matches_f32_pack(oracle, m, n, k):
    """src/cpu/gemm.rs:806-827: f16 panels of f16-rounded weights are bit-identical."""
    a = ((np.arange(m * k) % 19) * 0.013 - 0.11).astype(np.float32).reshape(m, k)
    w = oracle.round_f16(((np.arange(n * k) % 23) * 0.017 - 0.2).astype(np.float32).reshape(n, k))
    c32 = oracle.gemm(a, oracle.PackW(w, half=False))
    c16 = oracle.gemm(a, oracle.PackW(w, half=True))
    assert np.array_equal(c32.view(np.uint32), c16.view(np.uint32))


def test_gemm_unaligned_column_counts(oracle):
    """src/cpu/gemm.rs:833-851."""
    for ncols in range(60, 200, 7):
        m, k = ncols, 9
        a = ((np.arange(m * k) % 19) * 0.03 - 0.2).astype(np.float32).reshape(m, k)
        w = ((np.arange(ncols * k) % 23) * 0.02 - 0.15).astype(np.float32).reshape(ncols, k)
        assert np.max(np.abs(oracle.gemm(a, oracle.PackW(w)) - _naive(a, w))) < 1e-4


@pytest.mark.parametrize("m,n,k,threads", [(37, 53, 301, 3), (200, 130, 1024, 8), (6, 16, 4096, 1)])
def test_blocked_gemm_is_the_fma_chain(oracle, m, n, k, threads):
    """Each output of the blocked AVX2 kernel equals one fmaf chain over
    ascending k (src/cpu/gemm.rs:654-671), whatever the tiling / threads."""
    rng = np.random.default_rng(m * n)
    a = rng.standard_normal((m, k), dtype=np.float32)
    w = oracle.round_f16(rng.standard_normal((n, k), dtype=np.float32))
    want = oracle.gemm_fma_chain(a, w)
    for half in (False, True):
        got = oracle.gemm(a, oracle.PackW(w, half=half), threads=threads)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a column window starting on a panel boundary
    got = oracle.gemm(a, oracle.PackW(w), n0=16, ncols=n - 16)
    assert np.array_equal(got.view(np.uint32), want[:, 16:].view(np.uint32))


def test_split_k_partition(oracle):
    """src/cpu/gemm.rs:348-415: workers = min(w, ceil(k/64)); chunk =
    ceil(k/workers); partials are fma chains summed in worker order."""
    rng = np.random.default_rng(3)
    m, n, k, workers = 40, 128, 700, 5
    a = rng.random((m, k), dtype=np.float32)
    w = oracle.round_f16(rng.standard_normal((n, k), dtype=np.float32))
    got = oracle.gemm_split_k(a, oracle.PackW(w), workers)
    wk = min(workers, -(-k // 64))
    chunk = -(-k // wk)
    parts = [oracle.gemm_fma_chain(a[:, i * chunk:(i + 1) * chunk], w[:, i * chunk:(i + 1) * chunk]) for i in range(wk)]
    acc = np.zeros((m, n), np.float32)
    for p in parts:
        acc = (acc + p).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), acc.view(np.uint32))
    assert np.max(np.abs(got - _naive(a, w))) < 1e-3


# ------------------------------------------------------------------- row ops
def test_layer_norm_vs_f64(oracle):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((33, 1024), dtype=np.float32) * 3 + 1
    w = rng.standard_normal(1024, dtype=np.float32)
    b = rng.standard_normal(1024, dtype=np.float32)
    x64 = x.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    var = x64.var(1, keepdims=True)
    want = (x64 - mu) / np.sqrt(var + 1e-5) * w + b
    got = oracle.layer_norm(x, w, b)
    assert np.max(np.abs(got - want)) < 1e-4 * np.max(np.abs(want))


def test_layer_norm_constant_row_gives_bias(oracle):
    x = np.full((2, 1024), 3.25, np.float32)
    w = np.arange(1024, dtype=np.float32)
    b = np.linspace(-1, 1, 1024).astype(np.float32)
    assert np.array_equal(oracle.layer_norm(x, w, b), np.broadcast_to(b, (2, 1024)))


def test_silu_glu_closed_forms(oracle):
    x = np.linspace(-20, 20, 4001).astype(np.float32)
    want = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(oracle.silu(x) - want)) < 1e-5
    g = np.stack([np.linspace(-3, 3, 64), np.linspace(5, -5, 64)]).reshape(1, 128).astype(np.float32)
    a, gate = g[0, :64].astype(np.float64), g[0, 64:].astype(np.float64)
    assert np.max(np.abs(oracle.glu(g)[0] - a / (1 + np.exp(-gate)))) < 1e-6


def test_rel_softmax_shift_convention(oracle):
    """probs[q,k] = softmax_k(scale*(content[q,k] + bd[q, t-1-q+k])) —
    checked against the Transformer-XL pad/reshape _rel_shift formulation
    (transformers modeling_parakeet.py ParakeetEncoderAttention._rel_shift),
    a different algorithm for the same shift."""
    rng = np.random.default_rng(5)
    t = 37
    p = 2 * t - 1
    content = rng.standard_normal((t, t)).astype(np.float32)
    bd_full = rng.standard_normal((t, p)).astype(np.float32)  # column j <-> position t-1-j
    scale = 0.0883883461356163
    got = oracle.rel_softmax_rows(content, bd_full, p, t, 0, 0, scale)
    # pad-left / reshape / drop-first-row shift
    padded = np.pad(bd_full.astype(np.float64), ((0, 0), (1, 0)))
    shifted = padded.reshape(p + 1, t)[1:].reshape(t, p)[:, :t]
    s = scale * (content.astype(np.float64) + shifted)
    s = np.exp(s - s.max(1, keepdims=True))
    want = s / s.sum(1, keepdims=True)
    assert np.max(np.abs(got - want)) < 1e-6


def test_dwconv_bn_silu_vs_numpy(oracle):
    rng = np.random.default_rng(6)
    t, c = 21, 1024
    x = rng.standard_normal((t, c), dtype=np.float32)
    dw = rng.standard_normal((c, 9), dtype=np.float32) * 0.3
    a = rng.random(c, dtype=np.float32) + 0.5
    b = rng.standard_normal(c, dtype=np.float32) * 0.1
    xp = np.pad(x.astype(np.float64), ((4, 4), (0, 0)))
    y = sum(xp[i:i + t] * dw[:, i] for i in range(9)) * a + b
    want = y / (1 + np.exp(-y))
    assert np.max(np.abs(oracle.dwconv_bn_silu(x, dw, a, b) - want)) < 1e-5


def test_pos_embed(oracle):
    """src/encoder.rs:228-245: row pi <-> pos = T-1-pi, [2i]=sin, [2i+1]=cos of
    pos / 10000^(2i/1024); the pos = 0 row is exactly [0, 1, 0, 1, ...]."""
    t = 50
    got = oracle.pos_embed(t)
    pos = (t - 1 - np.arange(2 * t - 1))[:, None].astype(np.float64)
    inv = 1.0 / 10000 ** (np.arange(0, 1024, 2) / 1024.0)
    want = np.empty((2 * t - 1, 1024))
    want[:, 0::2], want[:, 1::2] = np.sin(pos * inv), np.cos(pos * inv)
    assert np.max(np.abs(got - want)) < 1e-4
    mid = got[t - 1]
    assert np.all(mid[0::2] == 0.0) and np.all(mid[1::2] == 1.0)
