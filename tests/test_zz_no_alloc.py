"""smk_d_gemm_q4_0_noalloc (no reference counterpart): the batched Q4_0 product with the
library's fixed scratch array instead of an allocated buffer.  Through the C ABI, two calls in a
row -- the second with fewer rows of x and a shorter K -- each equal smk_d_gemm_q4_0 bit for bit
(and so the reference's SIMD order, which the batched tests pin); a call whose x image would not
fit the array is refused with a clear error and writes nothing."""

import numpy as np
import pytest

from oracle import oracle as o
from simd_ml_kernels import abi
from tests import gpu_util as g

pytestmark = pytest.mark.gpu


def _gemm(entry, X, wq, N, K):
    M = X.shape[0]
    xd, wd = g.dev(X), g.dev(wq)
    yd = g.dev(np.full(M * N + 256, 0xEEEEEEEE, np.uint32))
    g.call(entry, M, N, K, g.ptr(xd), K, g.ptr(wd), g.ptr(yd), N, None)
    out = g.host(yd, np.uint32, M * N + 256)
    assert (out[M * N:] == 0xEEEEEEEE).all(), "wrote past Y"
    return out[:M * N].view(np.float32).reshape(M, N)


@pytest.mark.parametrize("order", ["noalloc_first", "allocating_first"])
def test_two_calls_equal_the_allocating_entry(order):
    rng = np.random.default_rng(71)
    cases = []
    for M, N, K in ((32, 1000, 4096), (5, 301, 2048)):   # the second smaller: rows, N and K
        X = rng.standard_normal((M, K)).astype(np.float32)
        wq = o.quantize_q4_0(rng.standard_normal((N, K)).astype(np.float32))
        cases.append((X, wq, N, K))
    for X, wq, N, K in cases:
        if order == "noalloc_first":
            Y0 = _gemm("smk_d_gemm_q4_0_noalloc", X, wq, N, K)
            Y1 = _gemm("smk_d_gemm_q4_0", X, wq, N, K)
        else:
            Y1 = _gemm("smk_d_gemm_q4_0", X, wq, N, K)
            Y0 = _gemm("smk_d_gemm_q4_0_noalloc", X, wq, N, K)
        np.testing.assert_array_equal(Y0.view(np.uint32), Y1.view(np.uint32))
        for m in (0, X.shape[0] - 1):
            np.testing.assert_array_equal(Y0[m].view(np.uint32), o.gemv_q4_0_simd(X[m], wq, N, K).view(np.uint32))


def test_rows_beyond_the_array_are_refused():
    """512 rows of K = 14336 need about 8 MiB of x image: refused, Y untouched (real buffers of
    the full size, so nothing could go out of bounds either way)."""
    M, N, K = 512, 64, 14336
    xd, wd = g.empty(4 * M * K, 0), g.empty(N * (K // 32) * 18, 0x88)
    yd = g.dev(np.full(M * N, 0xEEEEEEEE, np.uint32))
    L = abi.lib()
    rc = L.smk_d_gemm_q4_0_noalloc(M, N, K, g.ptr(xd), K, g.ptr(wd), g.ptr(yd), N, None)
    assert rc == abi.SMK_ERR_ARGUMENT
    assert "scratch" in L.smk_last_error().decode()
    assert (g.host(yd, np.uint32, M * N) == 0xEEEEEEEE).all()
