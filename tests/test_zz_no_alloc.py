"""bark_hip_lowbit_linear_noalloc through the C ABI: the same results as
bark_hip_lowbit_linear (same kernels, so bit-identical) on two calls in a row,
the second with a smaller input, for shapes that split K (the partial sums sit
in the fixed per-GPU scratch array) and one that does not; the scratch keeps
the previous call's contents, which must not leak into the next result.
A shape whose partial sums exceed the scratch is rejected with an error."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _case(rng, t, k, n):
    a = torch.from_numpy(rng.standard_normal((t, k), dtype=np.float32)).to(torch.bfloat16).cuda()
    codes = torch.from_numpy(rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)).cuda()
    lut = np.sort(rng.standard_normal((n, 16), dtype=np.float32) * 0.02, axis=1).astype(np.float16)
    lut_d = torch.from_numpy(lut.view(np.uint16).view(np.int16)).cuda()
    return a, codes, lut_d


def _run(pkg, fn, a, codes, lut, t, k, n):
    c = torch.full((t, n), float("nan"), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    fn(a.data_ptr(), 1, codes.data_ptr(), lut.data_ptr(), c.data_ptr(), 0, t, k, n, s)
    torch.cuda.synchronize()
    return c.cpu().numpy()


@pytest.mark.parametrize("k,n,ts", [(1024, 4096, (188, 61)), (4096, 1024, (2207, 900)), (1024, 3072, (700, 33))])
def test_noalloc_equals_lowbit_linear(pkg, k, n, ts):
    rng = np.random.default_rng(k + n)
    for t in ts:  # the second call is smaller than the first
        print(f"case noalloc t={t} k={k} n={n}", flush=True)
        a, codes, lut = _case(rng, t, k, n)
        want = _run(pkg, pkg.lowbit_linear, a, codes, lut, t, k, n)
        got = _run(pkg, pkg.lowbit_linear_noalloc, a, codes, lut, t, k, n)
        assert np.isfinite(want).all()
        assert np.array_equal(got, want)


def test_noalloc_rejects_oversized_scratch(pkg):
    """T = 3500, K = 4096, N = 1024 splits K in two: 2 x 3500 x 1024 x 4
    bytes (28.7 MB) of partial sums exceed the 24 MiB scratch; nothing is
    launched and the error names the limit."""
    t, k, n = 3500, 4096, 1024
    a = torch.zeros((t, k), dtype=torch.bfloat16, device="cuda")
    codes = torch.zeros((n, k // 2), dtype=torch.uint8, device="cuda")
    lut = torch.zeros((n, 16), dtype=torch.int16, device="cuda")
    c = torch.zeros((t, n), dtype=torch.float32, device="cuda")
    with pytest.raises(pkg.HipError, match="scratch"):
        pkg.lowbit_linear_noalloc(a.data_ptr(), 1, codes.data_ptr(), lut.data_ptr(), c.data_ptr(), 0, t, k, n,
                                  torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
