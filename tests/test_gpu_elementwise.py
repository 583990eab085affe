"""GPU parity of the kernels around the decode GEMVs, through the C ABI.

  * RMSNorm and RoPE restate examples/llama/llama.py's numpy code (:184-187, :387-396,
    :169-178) and must equal it bit for bit (numpy evaluates the oracle in this process);
  * SiLU: bit-exact with the reference's SIMD tables (silu_avx2.cpp:38-45 and its exp,
    simd_math.hpp:63-117, restated in the oracle and pinned to the reference build), hence
    within its bound 1e-35 + 1e-6 |y64| (activations.hpp:20-23) with its special values;
  * softmax rows: bit-exact with softmax_row_avx2 (the same way), within its stated 5e-6 of the
    float64 softmax (softmax_avx2.cpp:24-27), NaN rows as its non-finite rules;
  * FP32/FP16/BF16 trans_b products: |C - C64| <= 2(K+2)u (|A||W|^T) (test_precision.py:212-220).
"""

import math

import numpy as np
import pytest

from oracle import oracle as o
from tests import gpu_util as g

pytestmark = pytest.mark.gpu

RMS_WIDTHS = [1, 5, 7, 8, 9, 64, 100, 128, 129, 136, 200, 260, 300, 1000, 2048, 3072, 4096, 5120, 8192, 8193,
              11008, 14336, 16384, 20000, 40000]


def d_rms_norm(x, w, eps):
    rows, n = x.shape
    xd, wd, yd = g.dev(x), g.dev(w), g.empty(4 * rows * n + 64)
    g.call("smk_d_rms_norm", g.ptr(xd), g.ptr(wd), g.ptr(yd), rows, n, eps, g.stream())
    out = g.host(yd, np.float32, rows * n + 16)
    assert (out[rows * n:].view(np.uint32) == 0xEEEEEEEE).all(), "wrote past y"
    return out[:rows * n].reshape(rows, n)


class TestRmsNorm:
    @pytest.mark.parametrize("n", RMS_WIDTHS)
    def test_bit_exact_with_numpy(self, n):
        rng = np.random.default_rng(n)
        rows = 3
        x = np.stack([(rng.standard_normal(n) * 10.0 ** s).astype(np.float32) for s in (-3, 0, 3)])
        w = rng.standard_normal(n).astype(np.float32)
        for eps in (1e-5, 1e-6):
            y = d_rms_norm(x, w, eps)
            for r in range(rows):
                ref = o.rms_norm(x[r], w, eps)
                np.testing.assert_array_equal(y[r].view(np.uint32), ref.view(np.uint32), err_msg=f"n={n} row {r}")

    def test_llama_widths_many_rows(self):
        """hidden 2048 (Llama-3.2-1B) and 4096 (Llama-3-8B): 64 rows of residual-like values."""
        rng = np.random.default_rng(7)
        for n in (2048, 4096):
            x = (rng.standard_normal((64, n)) * rng.uniform(0.01, 50, (64, 1))).astype(np.float32)
            w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
            y = d_rms_norm(x, w, 1e-5)
            ref = np.stack([o.rms_norm(x[r], w, 1e-5) for r in range(64)])
            np.testing.assert_array_equal(y.view(np.uint32), ref.view(np.uint32))

    def test_zero_row_and_specials(self):
        n = 2048
        x = np.zeros((3, n), np.float32)
        x[1, 5] = np.inf
        x[2, 7] = np.nan
        w = np.ones(n, np.float32)
        y = d_rms_norm(x, w, 1e-5)
        with np.errstate(invalid="ignore", over="ignore"):
            ref = np.stack([o.rms_norm(x[r], w, 1e-5) for r in range(3)])
        np.testing.assert_array_equal(np.isnan(y), np.isnan(ref))
        fin = ~np.isnan(ref)
        np.testing.assert_array_equal(y[fin].view(np.uint32), ref[fin].view(np.uint32))


class TestRope:
    @pytest.mark.parametrize("interleaved", [True, False])
    @pytest.mark.parametrize("heads,hd", [(32, 64), (8, 64), (32, 128), (3, 2)])
    def test_bit_exact_with_numpy(self, interleaved, heads, hd):
        rng = np.random.default_rng(heads * hd)
        inv = o.rope_inv_freq(hd, 500000.0, {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                             "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})
        for pos in (0, 1, 17, 1000, 131071):
            cos, sin = o.rope_cos_sin(inv, pos)
            x = (rng.standard_normal((heads, hd)) * 3).astype(np.float32)
            xd, cd, sd, yd = g.dev(x), g.dev(cos), g.dev(sin), g.empty(4 * heads * hd)
            g.call("smk_d_rope", g.ptr(xd), g.ptr(cd), g.ptr(sd), g.ptr(yd), heads, hd, int(interleaved), g.stream())
            y = g.host(yd, np.float32, heads * hd).reshape(heads, hd)
            ref = o.rope(x, cos, sin, interleaved)
            np.testing.assert_array_equal(y.view(np.uint32), ref.view(np.uint32), err_msg=f"pos {pos}")

    def test_in_place(self):
        heads, hd = 32, 64
        rng = np.random.default_rng(1)
        cos, sin = o.rope_cos_sin(o.rope_inv_freq(hd, 500000.0, None), 33)
        x = rng.standard_normal((heads, hd)).astype(np.float32)
        xd, cd, sd = g.dev(x), g.dev(cos), g.dev(sin)
        g.call("smk_d_rope", g.ptr(xd), g.ptr(cd), g.ptr(sd), g.ptr(xd), heads, hd, 1, g.stream())
        y = g.host(xd, np.float32, heads * hd).reshape(heads, hd)
        np.testing.assert_array_equal(y.view(np.uint32), o.rope(x, cos, sin, True).view(np.uint32))


def d_unary(name, x, *extra):
    xd, yd = g.dev(x), g.empty(x.nbytes + 64)
    g.call(name, g.ptr(xd), g.ptr(yd), *extra, g.stream())
    out = g.host(yd, np.float32, x.size + 16)
    assert (out[x.size:].view(np.uint32) == 0xEEEEEEEE).all(), "wrote past the output"
    return out[:x.size].reshape(x.shape)


class TestSilu:
    def test_within_reference_bound(self):
        rng = np.random.default_rng(0)
        x = np.concatenate([rng.standard_normal(1 << 16) * 8, rng.uniform(-100, 100, 1 << 14),
                            np.linspace(-90, 30, 4001)]).astype(np.float32)
        y = d_unary("smk_d_silu", x, x.size)
        ref = o.silu64(x)
        assert (np.abs(y - ref) <= 1e-35 + 1e-6 * np.abs(ref)).all()

    def test_special_values(self):
        x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -88.0, -88.5, -89.0, -100.0, -1e30, 1e30, 88.7],
                     np.float32)
        y = d_unary("smk_d_silu", x, x.size)
        assert y[0] == 0 and y[1] == 0
        assert y[2] == np.inf and np.isnan(y[3]) and np.isnan(y[4])
        for v, yy in zip(x[6:10], y[6:10]):  # -x > 88: the denominator is +inf, the result -0
            assert yy == 0 and np.signbit(yy), v
        assert y[10] == np.float32(1e30)
        ref = o.silu64(x[5:6])
        assert abs(y[5] - ref[0]) <= 1e-35 + 1e-6 * abs(ref[0])

    def test_bit_exact_with_reference_simd(self):
        """silu_avx2's arithmetic (the reference's SIMD tables), restated in the oracle and pinned
        there to the reference build."""
        rng = np.random.default_rng(4)
        x = np.concatenate([rng.standard_normal(1 << 16) * 10, rng.uniform(-120, 120, 1 << 14),
                            np.array([0, -0.0, 88, -88, 88.5, -88.5, 1e30, -1e30, np.inf, -np.inf, np.nan])]).astype(np.float32)
        y = d_unary("smk_d_silu", x, x.size)
        ref = o.silu_simd(x)
        np.testing.assert_array_equal(np.isnan(y), np.isnan(ref))
        fin = ~np.isnan(ref)
        np.testing.assert_array_equal(y[fin].view(np.uint32), ref[fin].view(np.uint32))

    def test_matches_oracle_scalar(self):
        rng = np.random.default_rng(3)
        x = (rng.standard_normal(8192) * 10).astype(np.float32)
        y = d_unary("smk_d_silu", x, x.size)
        ref = o.silu_scalar(x).astype(np.float64)
        assert (np.abs(y - ref) <= 2e-6 * np.abs(ref) + 1e-35).all()


class TestSoftmax:
    @pytest.mark.parametrize("rows,n", [(1, 1), (3, 7), (4, 64), (5, 1000), (2, 4097), (32, 161)])
    def test_close_to_float64(self, rows, n):
        rng = np.random.default_rng(rows * n)
        x = (rng.standard_normal((rows, n)) * 5).astype(np.float32)
        y = d_unary("smk_d_softmax", x, rows, n)
        ref = o.softmax64(x)
        assert (np.abs(y - ref) <= 5e-6).all()
        assert np.allclose(y.sum(axis=1), 1.0, atol=1e-5)

    @pytest.mark.parametrize("n", [1, 5, 8, 9, 16, 33, 127, 160, 1000])
    def test_bit_exact_with_reference_simd(self, n):
        """softmax_row_avx2's order; the tail's double exp is the device's (one double ulp from
        glibc's), so equality is expected but not guaranteed for the last n % 8 values."""
        rng = np.random.default_rng(n)
        x = (rng.standard_normal((6, n)) * rng.uniform(0.5, 10, (6, 1))).astype(np.float32)
        y = d_unary("smk_d_softmax", x, 6, n)
        np.testing.assert_array_equal(y.view(np.uint32), o.softmax_simd(x).view(np.uint32))

    def test_nan_rules(self):
        x = np.zeros((4, 16), np.float32)
        x[0, 3] = np.nan
        x[1, 2] = np.inf
        x[2, :] = -np.inf
        x[3, 5] = -np.inf
        y = d_unary("smk_d_softmax", x, 4, 16)
        assert np.isnan(y[:3]).all()
        assert y[3, 5] == 0 and np.allclose(y[3].sum(), 1.0)


def _lowp_operands(fmt, M, N, K, rng):
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if fmt == "fp32":
        return A, W, A, W
    if fmt == "f16":
        a16, w16 = A.astype(np.float16), W.astype(np.float16)
        return a16.view(np.uint16), w16.view(np.uint16), a16.astype(np.float32), w16.astype(np.float32)
    ab, wb = o.to_bf16_rne(A), o.to_bf16_rne(W)
    return ab, wb, o.bf16_to_f32(ab), o.bf16_to_f32(wb)


ELEM = {"fp32": 0, "f16": 1, "bf16": 2}


def d_gemm_tb(fmt, A, W, M, N, K, alpha=1.0, beta=0.0, C=None, ldb=None, b_offset=0):
    ldb = K if ldb is None else ldb
    es = A.itemsize
    ad = g.dev(A)
    staged = np.zeros(b_offset + N * ldb * es + 64, np.uint8)
    Wb = np.zeros((N, ldb), W.dtype)
    Wb[:, :K] = W
    staged[b_offset:b_offset + Wb.nbytes] = Wb.view(np.uint8).reshape(-1)
    wd = g.dev(staged)
    c0 = np.zeros((M, N), np.float32) if C is None else C
    cd = g.dev(c0)
    g.call("smk_d_gemm_tb", ELEM[fmt], M, N, K, alpha, g.ptr(ad), K, g.ptr(wd, b_offset), ldb, beta, g.ptr(cd), N,
           g.stream())
    return g.host(cd, np.float32, M * N).reshape(M, N)


class TestGemmTb:
    @pytest.mark.parametrize("fmt", ["fp32", "f16", "bf16"])
    @pytest.mark.parametrize("M,N,K", [(1, 1, 8), (1, 300, 2048), (2, 129, 4096), (3, 64, 520), (8, 96, 1024),
                                       (1, 17, 13), (5, 33, 100), (9, 40, 256)])
    def test_within_bound(self, fmt, M, N, K):
        rng = np.random.default_rng(M * 1000 + N + K)
        A, W, A32, W32 = _lowp_operands(fmt, M, N, K, rng)
        C = d_gemm_tb(fmt, A, W, M, N, K)
        A64, W64 = A32.astype(np.float64), W32.astype(np.float64)
        ref = A64 @ W64.T
        bound = o.gemm_bound(K, np.abs(A64) @ np.abs(W64).T)
        assert (np.abs(C - ref) <= bound + 1e-300).all()

    @pytest.mark.parametrize("fmt", ["fp32", "f16", "bf16"])
    def test_alpha_beta(self, fmt):
        M, N, K = 2, 70, 512
        rng = np.random.default_rng(5)
        A, W, A32, W32 = _lowp_operands(fmt, M, N, K, rng)
        C0 = rng.standard_normal((M, N)).astype(np.float32)
        C = d_gemm_tb(fmt, A, W, M, N, K, alpha=0.5, beta=2.0, C=C0)
        A64, W64 = A32.astype(np.float64), W32.astype(np.float64)
        ref = 2.0 * C0.astype(np.float64) + 0.5 * (A64 @ W64.T)
        bound = 0.5 * o.gemm_bound(K, np.abs(A64) @ np.abs(W64).T) + 4 * 2.0 ** -24 * np.abs(ref)
        assert (np.abs(C - ref) <= bound).all()

    @pytest.mark.parametrize("fmt", ["fp32", "f16", "bf16"])
    def test_unaligned_and_padded_rows(self, fmt):
        """Rows of W with a leading dimension > K and a 2-byte offset take the plain kernel."""
        M, N, K = 1, 50, 256
        rng = np.random.default_rng(9)
        A, W, A32, W32 = _lowp_operands(fmt, M, N, K, rng)
        for ldb, off in ((K + 8, 0), (K, 2 if fmt != "fp32" else 4)):
            C = d_gemm_tb(fmt, A, W, M, N, K, ldb=ldb, b_offset=off)
            A64, W64 = A32.astype(np.float64), W32.astype(np.float64)
            ref = A64 @ W64.T
            assert (np.abs(C - ref) <= o.gemm_bound(K, np.abs(A64) @ np.abs(W64).T) + 1e-300).all()

    def test_nan_in_x_row_gives_nan_row(self):
        M, N, K = 3, 40, 256
        rng = np.random.default_rng(2)
        A = rng.standard_normal((M, K)).astype(np.float32)
        A[1, 17] = np.nan
        W = rng.standard_normal((N, K)).astype(np.float32)
        C = d_gemm_tb("fp32", A, W, M, N, K)
        assert np.isnan(C[1]).all() and not np.isnan(C[[0, 2]]).any()

    def test_k_zero_scales_c(self):
        C0 = np.arange(12, dtype=np.float32).reshape(3, 4)
        A = np.zeros((3, 1), np.float32)
        W = np.zeros((4, 1), np.float32)
        C = d_gemm_tb("fp32", A, W, 3, 4, 0, beta=0.5, C=C0)
        np.testing.assert_array_equal(C, C0 * np.float32(0.5))


class TestSgemm:
    @pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
    def test_transposes(self, ta, tb):
        M, N, K = 5, 33, 70
        rng = np.random.default_rng(ta * 2 + tb)
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.standard_normal((K, N)).astype(np.float32)
        Ast = np.ascontiguousarray(A.T) if ta else A
        Bst = np.ascontiguousarray(B.T) if tb else B
        ad, bd, cd = g.dev(Ast), g.dev(Bst), g.dev(np.zeros((M, N), np.float32))
        lda = M if ta else K
        ldb = K if tb else N
        g.call("smk_d_sgemm", ta, tb, M, N, K, 1.0, g.ptr(ad), lda, g.ptr(bd), ldb, 0.0, g.ptr(cd), N, g.stream())
        C = g.host(cd, np.float32, M * N).reshape(M, N)
        A64, B64 = A.astype(np.float64), B.astype(np.float64)
        bound = o.gemm_bound(K, np.abs(A64) @ np.abs(B64))
        assert (np.abs(C - A64 @ B64) <= bound).all()

    def test_attention_shapes(self):
        """The example's attention calls: scores = scale q K^T, then p V (llama.py:398-412)."""
        rep, hd, T = 4, 64, 77
        rng = np.random.default_rng(11)
        q = rng.standard_normal((rep, hd)).astype(np.float32)
        Kc = rng.standard_normal((T, hd)).astype(np.float32)
        V = rng.standard_normal((T, hd)).astype(np.float32)
        scale = 1.0 / math.sqrt(hd)
        qd, kd, vd = g.dev(q), g.dev(Kc), g.dev(V)
        sd = g.dev(np.zeros((rep, T), np.float32))
        g.call("smk_d_sgemm", 0, 1, rep, T, hd, scale, g.ptr(qd), hd, g.ptr(kd), hd, 0.0, g.ptr(sd), T, g.stream())
        S = g.host(sd, np.float32, rep * T).reshape(rep, T)
        ref = scale * (q.astype(np.float64) @ Kc.astype(np.float64).T)
        assert (np.abs(S - ref) <= scale * o.gemm_bound(hd, np.abs(q).astype(np.float64) @ np.abs(Kc).T) +
                4 * 2.0 ** -24 * np.abs(ref)).all()
        P = o.softmax64(S).astype(np.float32)
        pd, od = g.dev(P), g.dev(np.zeros((rep, hd), np.float32))
        g.call("smk_d_sgemm", 0, 0, rep, hd, T, 1.0, g.ptr(pd), T, g.ptr(vd), hd, 0.0, g.ptr(od), hd, g.stream())
        Out = g.host(od, np.float32, rep * hd).reshape(rep, hd)
        ref2 = P.astype(np.float64) @ V.astype(np.float64)
        assert (np.abs(Out - ref2) <= o.gemm_bound(T, np.abs(P).astype(np.float64) @ np.abs(V))).all()
