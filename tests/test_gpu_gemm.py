"""GPU parity of the 4-bit level-table linear through the
C ABI entry point bark_hip_lowbit_linear."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _lut4(rng, n, k):
    codes = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    lut = np.sort(rng.standard_normal((n, 16), dtype=np.float32) * 0.02, axis=1).astype(np.float16)
    return codes, lut


def _weights(codes, lut):
    lo = (codes & 15).astype(np.intp)
    hi = (codes >> 4).astype(np.intp)
    idx = np.empty((codes.shape[0], codes.shape[1] * 2), np.intp)
    idx[:, 0::2], idx[:, 1::2] = lo, hi
    return np.take_along_axis(lut.astype(np.float32), idx, axis=1)


def _bf16(x: np.ndarray) -> np.ndarray:
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return u


def _run(pkg, a_bits, a_dtype, codes, lut, c_dtype, t, k, n):
    A = _dev(a_bits)
    C = torch.empty((t, n), dtype=torch.float32 if c_dtype == 0 else torch.int16, device="cuda")
    dc, dl = _dev(codes), _dev(lut.view(np.uint16))
    pkg.lowbit_linear(A.data_ptr(), a_dtype, dc.data_ptr(), dl.data_ptr(), C.data_ptr(), c_dtype, t, k, n,
                      torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    out = C.cpu().numpy()
    if c_dtype == 2:
        out = (out.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    elif c_dtype == 1:
        out = out.view(np.float16).astype(np.float32)
    return out


@pytest.mark.parametrize("t", [188, 2207])
@pytest.mark.parametrize("k,n", [(1024, 4096), (4096, 1024), (1024, 3072)])
def test_lowbit_linear_config1(pkg, t, k, n):
    """bf16 activations, bf16 out, f32 accumulate (config 1) vs an f64 product
    of the same bf16 activations and the exact f16 level values."""
    print(f"case lowbit_linear t={t} k={k} n={n}", flush=True)
    rng = np.random.default_rng([t, k, n])
    a = rng.standard_normal((t, k), dtype=np.float32)
    a_bits = _bf16(a)
    a_val = (a_bits.astype(np.uint32) << 16).view(np.float32)
    codes, lut = _lut4(rng, n, k)
    w = _weights(codes, lut)
    ref = a_val.astype(np.float64) @ w.astype(np.float64).T
    got = _run(pkg, a_bits, 1, codes, lut, 2, t, k, n)
    scale = np.max(np.abs(ref))
    # bf16 output rounding (2^-9 relative) plus f32 accumulation
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-8 + 1e-4 * scale)
    got32 = _run(pkg, a_bits, 1, codes, lut, 0, t, k, n)
    assert np.max(np.abs(got32 - ref)) <= 2e-5 * scale


def test_lowbit_dequant_bit_exact(pkg):
    """With A = identity the product returns W^T exactly (one nonzero term per
    output), so every code->level expansion is checked bit for bit."""
    k, n = 1024, 256
    rng = np.random.default_rng(11)
    codes, lut = _lut4(rng, n, k)
    eye = np.eye(k, dtype=np.float16).view(np.uint16)
    got = _run(pkg, eye, 0, codes, lut, 0, k, k, n)
    want = _weights(codes, lut).T
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("t", [1, 63, 65, 130])
def test_lowbit_linear_ragged_rows(pkg, t):
    """Row counts that are not a multiple of the 64/128-row tile."""
    k, n = 1024, 256
    rng = np.random.default_rng([t, 5])
    a = rng.standard_normal((t, k), dtype=np.float32).astype(np.float16)
    codes, lut = _lut4(rng, n, k)
    ref = a.astype(np.float64) @ _weights(codes, lut).astype(np.float64).T
    got = _run(pkg, a.view(np.uint16), 0, codes, lut, 0, t, k, n)
    assert np.max(np.abs(got - ref)) <= 2e-5 * np.max(np.abs(ref))
