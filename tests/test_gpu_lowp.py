"""GPU parity of the FP32 / FP16 / BF16 decode GEMV (x @ W.T, W stored [N, K]) at BASELINE
config 3's Llama-3-8B shapes and at the reference's own trans_b cases.

Bar (the reference's, test_precision.py:205-220): both widenings to FP32 are exact, so the
reference value is the float64 product of the widened inputs and
|C - C64| <= 2(K+2)u * (|A||W|^T), u = 2^-24.  NaN in a row of W makes exactly that output NaN
(test_precision.py:238-250).  Both entry points are covered: the device entry smk_d_gemm_tb and
the pybind11 module's sgemm / sgemm_f16 / sgemm_bf16(trans_b=True) on host arrays (the host
slots of the KernelTable, including C with alpha and beta).
"""

import numpy as np
import pytest

from oracle import oracle as o
from tests import gpu_util as g

pytestmark = pytest.mark.gpu

ELEM = {"fp32": 0, "f16": 1, "bf16": 2}


def _as_fmt(x32: np.ndarray, fmt: str):
    """(array the kernel takes, its exact float64 values)."""
    if fmt == "fp32":
        return x32, x32.astype(np.float64)
    if fmt == "f16":
        h = x32.astype(np.float16)
        return h, h.astype(np.float64)
    b = o.to_bf16_rne(x32)
    return b, o.bf16_to_f32(b).astype(np.float64)


def _operands(fmt, M, N, K, seed, wscale=1.0):
    rng = np.random.default_rng(seed)
    A32 = rng.standard_normal((M, K), dtype=np.float32)
    W32 = rng.standard_normal((N, K), dtype=np.float32)
    if wscale != 1.0:
        W32 *= np.float32(wscale)
    (A, A64), (W, W64) = _as_fmt(A32, fmt), _as_fmt(W32, fmt)
    return A, A64, W, W64


def _device(fmt, A, W, M, N, K, alpha=1.0, beta=0.0, C=None):
    ad, wd = g.dev(A), g.dev(W)
    c0 = np.zeros((M, N), np.float32) if C is None else C.astype(np.float32)
    cd = g.dev(c0)
    g.call("smk_d_gemm_tb", ELEM[fmt], M, N, K, alpha, g.ptr(ad), K, g.ptr(wd), K, beta, g.ptr(cd), N, g.stream())
    return g.host(cd, np.float32, M * N).reshape(M, N)


def _check(C, A64, W64, K, alpha=1.0, beta=0.0, C0=None):
    ref = alpha * (A64 @ W64.T)
    mag = abs(alpha) * (np.abs(A64) @ np.abs(W64).T)
    if C0 is not None and beta != 0.0:
        ref = ref + beta * C0.astype(np.float64)
        mag = mag + abs(beta) * np.abs(C0.astype(np.float64))
    err = np.abs(C.astype(np.float64) - ref)
    bound = o.gemm_bound(K, mag)
    assert (err <= bound).all(), f"max err/bound {float(np.max(err / np.maximum(bound, 1e-300))):.3g}"


class TestConfig3Shapes:
    """x fp32 [1, K] ~ N(0,1), W ~ N(0, 0.02) cast to the weight type, fp32
    accumulation, at the Llama-3-8B FFN up/gate, down and attention-out shapes.  K = 14336 runs the
    64-lanes-per-row kernel (more than 512 groups of 8 elements), K = 4096 the 32-lane one."""

    @pytest.mark.parametrize("fmt", ["f16", "bf16", "fp32"])
    @pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336), (4096, 4096)])
    def test_within_bound(self, fmt, N, K):
        A, A64, W, W64 = _operands(fmt, 1, N, K, seed=N + K + ELEM[fmt], wscale=0.02)
        C = _device(fmt, A, W, 1, N, K)
        _check(C, A64, W64, K)

    @pytest.mark.parametrize("fmt", ["f16", "bf16"])
    def test_every_lane_split_kernel(self, fmt):
        """Row lengths that take each lane split of the streaming kernel: K = 8 (8 lanes),
        K = 200 (16 lanes, 25 groups), K = 4096 (32 lanes), K = 4104 (64 lanes, 513 groups), and
        several rows of x (M = 2, 4, 8) at K = 14336."""
        for M, N, K in ((1, 70, 8), (1, 513, 200), (1, 1000, 4096), (1, 999, 4104), (2, 300, 14336),
                        (4, 129, 14336), (8, 65, 14336)):
            A, A64, W, W64 = _operands(fmt, M, N, K, seed=M * 7 + N + K)
            C = _device(fmt, A, W, M, N, K)
            _check(C, A64, W64, K)

    @pytest.mark.parametrize("fmt", ["fp32", "f16", "bf16"])
    def test_nan_in_w_row_at_config_shape(self, fmt):
        """A NaN in one row of W (deep in K) makes exactly that output NaN, at 4096 x 14336."""
        N, K, j0 = 4096, 14336, 1234
        A, A64, W, W64 = _operands(fmt, 1, N, K, seed=5, wscale=0.02)
        W = W.copy()
        W[j0, K - 3] = {"fp32": np.float32(np.nan), "f16": np.float16(np.nan), "bf16": np.uint16(0x7FC0)}[fmt]
        C = _device(fmt, A, W, 1, N, K)
        assert np.isnan(C[0, j0])
        others = np.delete(C[0], j0)
        assert not np.isnan(others).any()
        _check(np.delete(C, j0, axis=1), A64, np.delete(W64, j0, axis=0), K)


class TestModuleTransB:
    """The reference's trans_b cases (test_precision.py:205-220) through the module's host entry
    points (sgemm, sgemm_f16, sgemm_bf16 with trans_b=True): the KernelTable slots on the GPU."""

    CASES = [(1, 37, 1), (1, 37, 15), (1, 37, 17), (1, 37, 33), (1, 1, 70), (1, 3, 70), (1, 5, 70),
             (1, 4096, 300), (1, 64, 4099), (1, 17, 70), (4, 33, 1027), (8, 45, 133), (9, 45, 133),
             (97, 113, 769), (1, 4096, 4096)]

    @staticmethod
    def _fn(fmt):
        import simd_ml_kernels as sk
        return {"fp32": sk.sgemm, "f16": sk.sgemm_f16, "bf16": sk.sgemm_bf16}[fmt]

    @pytest.mark.parametrize("fmt", ["fp32", "f16", "bf16"])
    @pytest.mark.parametrize("M,N,K", CASES)
    def test_trans_b_vs_float64(self, fmt, M, N, K):
        A, A64, W, W64 = _operands(fmt, M, N, K, seed=M * 1000 + N * 7 + K)
        C = self._fn(fmt)(A, W, trans_b=True)
        assert C.dtype == np.float32 and C.shape == (M, N)
        _check(C, A64, W64, K)

    @pytest.mark.parametrize("fmt", ["fp32", "f16", "bf16"])
    def test_unaligned_rows_alpha_beta_given_c(self, fmt):
        """x and W one element past an aligned address, C given with alpha = -1.5, beta = 0.5
        (test_precision.py:222-236); and the same with a larger C than x, so that the two host
        uploads of one call (x, then C) are both in flight before the product runs."""
        for M, N, K in ((1, 21, 77), (1, 4096, 64), (3, 1500, 40)):
            A, A64, W, W64 = _operands(fmt, M, N, K, seed=N + K)

            def shifted(v):
                buf = np.empty(v.size + 1, v.dtype)
                out = buf[1:].reshape(v.shape)
                out[...] = v
                return out

            A1, W1 = shifted(A), shifted(W)
            assert A1.ctypes.data % 8 != 0 and W1.ctypes.data % 8 != 0
            y0 = np.random.default_rng(K).standard_normal((M, N)).astype(np.float32)
            y = y0.copy()
            self._fn(fmt)(A1, W1, C=y, alpha=-1.5, beta=0.5, trans_b=True)
            _check(y, A64, W64, K, alpha=-1.5, beta=0.5, C0=y0)

    @pytest.mark.parametrize("fmt", ["fp32", "f16", "bf16"])
    def test_nan_propagates(self, fmt):
        """A NaN in row j0 of W (inside the K tail) makes exactly y[:, j0] NaN (test_precision.py:238-250)."""
        M, N, K, j0 = 1, 9, 45, 6
        A, _ = _as_fmt(np.full((M, K), 0.5, np.float32), fmt)
        Wf = np.full((N, K), 0.25, np.float32)
        Wf[j0, K - 2] = np.nan
        W, _ = _as_fmt(Wf, fmt)
        y = self._fn(fmt)(A, W, trans_b=True)
        assert np.isnan(y[:, j0]).all()
        assert (np.delete(y, j0, axis=1) == 0.125 * K).all()

    def test_config_3_shape_through_module(self):
        """FP16 at 14336 x 4096 through sgemm_f16(trans_b=True) with a read-only W (the pinned,
        device-resident weight path) equals the device entry point bit for bit."""
        N, K = 14336, 4096
        A, A64, W, W64 = _operands("f16", 1, N, K, seed=3, wscale=0.02)
        W.setflags(write=False)
        C = self._fn("f16")(A, W, trans_b=True)
        np.testing.assert_array_equal(C.view(np.uint32), _device("f16", A, W, 1, N, K).view(np.uint32))
        _check(C, A64, W64, K)
