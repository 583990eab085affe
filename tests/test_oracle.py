"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each oracle function is checked against something other than its own formula:
the committed llama.cpp v0.7.0 Q4_0 fixture, the known-answer blocks of the
reference's tests, closed forms (IEEE binary16 rounding, exhaustively), an
independent numpy restatement, the float64 exact sum with the reference's
documented bound, and -- where oracle/_ref was built from /root/reference --
the reference's own compiled kernels, bit for bit.  The last class plants
plausible mistakes in copies of the oracle and shows the checks catch them.
"""

import math
import os

import numpy as np
import pytest

from oracle import oracle as o

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
FIXTURE = os.path.join(GOLDEN, "q4_0_ggml_v0.7.0.npz")


def fixture_input() -> np.ndarray:
    """Input of the committed llama.cpp fixture, regenerated from its recipe
    (test_precision.py:640-664); the test checks it equals the stored copy."""
    rng = np.random.default_rng(2026)
    w = rng.standard_normal((20, 256)).astype(np.float32)
    w[:12] *= np.array([1, 3, 0.01, 100, 1e-3, 0.5, 7, 1, 1, 2, 40, 1e4], np.float32)[:, None]
    w[12] = np.tile(np.arange(-8, 8, 0.5, dtype=np.float32), 8)
    w[12, 32:64] = -w[12, 32:64]
    w[12, 64:] *= np.repeat(np.float32([0.25, 3, 1e-2, 7, 11, 0.125]), 32)
    w[13, :] = rng.uniform(-1, 1, 256).astype(np.float32)
    w[13, 5], w[13, 9] = 2.0, -2.0
    w[13, 35], w[13, 62] = -2.0, 2.0
    w[13, 64 + 20], w[13, 64 + 3] = 2.0, -2.0
    w[14, :32] = 0.0
    w[14, 32:64] = -0.0
    w[14, 64:96] = np.where(np.arange(32) % 3 == 0, 0.0, -0.0)
    w[15, :128] = rng.uniform(-1e-5, 1e-5, 128).astype(np.float32)
    w[15, 128:] = rng.uniform(-1e-36, 1e-36, 128).astype(np.float32)
    w[16, :] = rng.uniform(-5.2e5, 5.2e5, 256).astype(np.float32)
    w[17, :] = np.round(rng.uniform(-8, 8, 256)).astype(np.float32) * 0.5
    w[18, :] = -np.abs(w[18, :])
    w[19, ::2] = np.float32(7.0)
    w[19, 0::32] = np.float32(-8.0)
    return w


def q8_special_rows() -> np.ndarray:
    """Rows exercising every Q8_0 rule (test_precision.py:499-510)."""
    rng = np.random.default_rng(11)
    w = rng.standard_normal((6, 128)).astype(np.float32)
    w[0, :32] = np.arange(-16, 16) + 0.5
    w[0, 31] = 127.0
    w[1, :32] = 0.0
    w[1, 32:64] = rng.uniform(-1e-4, 1e-4, 32)
    w[2, :] = rng.uniform(-8.3e6, 8.3e6, 128)
    w[3, :32] = -w[3, :32]
    w[4, :32] = np.float32(1.0)
    w[5, :32] = np.where(np.arange(32) % 2, 1e-38, -1e-38).astype(np.float32)
    return w


# ─── fp16 ────────────────────────────────────────────────────────────────

class TestFp16:
    def test_every_half_round_trips_and_midpoints_round_to_even(self):
        L = o.lib()
        bad = 0
        for h in range(0x7C00):
            f = L.smko_fp16_to_fp32(h)
            bad += L.smko_fp32_to_fp16(f) != h
            bad += L.smko_fp32_to_fp16(-f) != (h | 0x8000)
            if h + 1 < 0x7C00:
                g = L.smko_fp16_to_fp32(h + 1)
                mid = np.float32((np.float64(f) + np.float64(g)) / 2)
                even = h + 1 if h & 1 else h
                bad += L.smko_fp32_to_fp16(float(mid)) != even
                bad += L.smko_fp32_to_fp16(float(np.nextafter(mid, np.float32(0)))) != h
                bad += L.smko_fp32_to_fp16(float(np.nextafter(mid, np.float32(1e9)))) != h + 1
        assert bad == 0

    def test_special_values(self):
        L = o.lib()
        u = lambda b: float(np.uint32(b).view(np.float32))
        assert L.smko_fp32_to_fp16(65519.996) == 0x7BFF
        assert L.smko_fp32_to_fp16(65520.0) == 0x7C00
        assert L.smko_fp32_to_fp16(u(0x7F800000)) == 0x7C00
        assert L.smko_fp32_to_fp16(u(0xFF800000)) == 0xFC00
        assert L.smko_fp32_to_fp16(u(0x7FC00001)) == 0x7E00
        assert L.smko_fp32_to_fp16(u(0xFFC00001)) == 0xFE00
        assert L.smko_fp32_to_fp16(1e-30) == 0
        assert L.smko_fp32_to_fp16(2.0 ** -25) == 0
        assert L.smko_fp32_to_fp16(float(np.nextafter(np.float32(2.0 ** -25), np.float32(1)))) == 1
        assert np.isnan(L.smko_fp16_to_fp32(0x7E00))
        assert L.smko_fp16_to_fp32(0xFC00) == -np.inf
        assert L.smko_fp16_to_fp32(0x8001) == -(2.0 ** -24)

    def test_matches_numpy_float16_on_random_floats(self):
        L = o.lib()
        rng = np.random.default_rng(7)
        bits = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)
        x = bits.view(np.float32)
        x = x[np.isfinite(x)]
        want = o.fp16_bits(x)
        got = np.array([L.smko_fp32_to_fp16(float(v)) for v in x], np.uint16)
        assert (got == want).all()

    def test_matches_reference_fp32_to_fp16(self, ref_lib):
        L = o.lib()
        rng = np.random.default_rng(8)
        bits = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)
        for v in bits.view(np.float32):
            assert L.smko_fp32_to_fp16(float(v)) == ref_lib.ref_fp32_to_fp16(float(v))


# ─── quantizers ──────────────────────────────────────────────────────────

class TestQ4_0Quantize:
    def test_llama_cpp_fixture(self):
        fx = np.load(FIXTURE, allow_pickle=False)
        np.testing.assert_array_equal(fx["w"], fixture_input())
        np.testing.assert_array_equal(o.quantize_q4_0(fx["w"]), fx["blocks"])
        np.testing.assert_array_equal(o.q4_0_quantize_numpy(fx["w"]), fx["blocks"])
        blk = fx["blocks"].reshape(20, 8, 18)
        assert blk[14, 0, :2].view("<u2")[0] == 0x8000 and (blk[14, 0, 2:] == 0x88).all()

    def test_special_blocks(self):
        w = np.zeros((2, 64), np.float32)
        w[0, :32] = np.where(np.arange(32) % 2, 1e-44, -1e-44).astype(np.float32)
        w[0, 32:] = 1.0
        w[1, :] = np.random.default_rng(1).standard_normal(64).astype(np.float32)
        q = o.quantize_q4_0(w)
        np.testing.assert_array_equal(q, o.q4_0_quantize_numpy(w))
        blk = q.reshape(2, 2, 18)
        assert (blk[0, 0, 2:] == 0x88).all() and blk[0, 0, :2].view("<f2")[0] == 0
        assert (blk[0, 1, 2:] == 0x00).all() and blk[0, 1, :2].view("<f2")[0] == np.float16(-0.125)

    @pytest.mark.parametrize("shape", [(32,), (1, 32), (7, 64), (33, 4096), (3, 2, 96)])
    def test_random_matches_numpy(self, shape):
        w = np.random.default_rng(sum(shape) + 1).standard_normal(shape).astype(np.float32) * 3
        np.testing.assert_array_equal(o.quantize_q4_0(w), o.q4_0_quantize_numpy(w))

    def test_rejects(self):
        for bad in (np.nan, np.inf, -np.inf):
            w = np.ones((1, 64), np.float32)
            w[0, 40] = bad
            with pytest.raises(ValueError):
                o.quantize_q4_0(w)
        w = np.ones((1, 64), np.float32)
        w[0, 3] = 8 * 65520.0
        with pytest.raises(ValueError):
            o.quantize_q4_0(w)
        w[0, 3] = 8 * 65504.0  # the largest scale is accepted
        o.quantize_q4_0(w)

    def test_matches_reference(self, ref_lib):
        w = np.concatenate([np.random.default_rng(6).standard_normal((40, 256)).astype(np.float32),
                            fixture_input()])
        got = o.quantize_q4_0(w)
        want = np.zeros_like(got)
        assert ref_lib.ref_quantize_q4_0(w.ctypes.data_as(o._f32p), w.shape[0], w.shape[1],
                                         want.ctypes.data_as(o._u8p)) == 1
        np.testing.assert_array_equal(got, want)


class TestQ8_0Quantize:
    def test_special_rows(self):
        w = q8_special_rows()
        q = o.quantize_q8_0(w)
        np.testing.assert_array_equal(q, o.q8_0_quantize_numpy(w))
        blk = q.reshape(6, 4, 34)
        assert blk[0, 0, 2:].view(np.int8).tolist()[:4] == [-16, -15, -14, -13]
        assert (blk[1, 0] == 0).all()
        assert (blk[4, 0, 2:].view(np.int8) == 127).all()
        assert (blk[5, 0, 2:] == 0).all() and blk[5, 0, :2].view("<f2")[0] == 0

    @pytest.mark.parametrize("shape", [(32,), (1, 32), (7, 64), (33, 4096), (3, 2, 96)])
    def test_random_matches_numpy(self, shape):
        w = np.random.default_rng(sum(shape)).standard_normal(shape).astype(np.float32) * 3
        np.testing.assert_array_equal(o.quantize_q8_0(w), o.q8_0_quantize_numpy(w))

    def test_rejects(self):
        w = np.ones((1, 64), np.float32)
        w[0, 40] = np.nan
        with pytest.raises(ValueError):
            o.quantize_q8_0(w)
        w = np.ones((1, 64), np.float32)
        w[0, 3] = 127 * 65520.0
        with pytest.raises(ValueError):
            o.quantize_q8_0(w)
        w[0, 3] = 127 * 65504.0
        o.quantize_q8_0(w)

    def test_matches_reference(self, ref_lib):
        w = np.concatenate([np.random.default_rng(5).standard_normal((40, 256)).astype(np.float32),
                            q8_special_rows()[:, :128].repeat(2, axis=1)])
        got = o.quantize_q8_0(w)
        want = np.zeros_like(got)
        assert ref_lib.ref_quantize_q8_0(w.ctypes.data_as(o._f32p), w.shape[0], w.shape[1],
                                         want.ctypes.data_as(o._u8p)) == 1
        np.testing.assert_array_equal(got, want)

    def test_x_quant_equals_weight_quants_with_fp32_scales(self, ref_lib):
        x = (np.random.default_rng(3).standard_normal(4096) * 4).astype(np.float32)
        x[:32] = np.arange(-16, 16) + 0.5
        qs, dx = o.quantize_x_q8(x)
        _, qw = o.q8_0_split(o.q8_0_quantize_numpy(x), 1, 4096)
        np.testing.assert_array_equal(qs, qw.reshape(-1))
        np.testing.assert_array_equal(dx, o.x_scales(x))
        rq = np.zeros(4096, np.int8)
        rd = np.zeros(128, np.float32)
        assert ref_lib.ref_quantize_x_q8(x.ctypes.data_as(o._f32p), 4096, rq.ctypes.data_as(o._i8p),
                                         rd.ctypes.data_as(o._f32p)) == 1
        np.testing.assert_array_equal(qs, rq)
        np.testing.assert_array_equal(dx.view(np.uint32), rd.view(np.uint32))
        x[100] = np.inf
        assert o.quantize_x_q8(x) is None


# ─── GEMV ────────────────────────────────────────────────────────────────

def _case(fmt, N, K, seed):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((N, K)).astype(np.float32)
    x = (rng.standard_normal(K) * 4).astype(np.float32)
    wq = (o.quantize_q4_0 if fmt == "q4_0" else o.quantize_q8_0)(w)
    return x, wq


SHAPES = [(1, 32), (7, 64), (8, 96), (9, 128), (17, 352), (100, 4096), (33, 11008)]


class TestGemv:
    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    def test_block_sums_exact(self, fmt):
        N, K = 17, 352
        x, wq = _case(fmt, N, K, 1)
        qs, _ = o.quantize_x_q8(x)
        got = o.block_sums(fmt, qs, wq, N, K)
        _, qw = (o.q4_0_split if fmt == "q4_0" else o.q8_0_split)(wq, N, K)
        want = (qw.astype(np.int64) * qs.reshape(1, K // 32, 32).astype(np.int64)).sum(axis=2)
        np.testing.assert_array_equal(got, want)

    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    @pytest.mark.parametrize("N,K", SHAPES)
    def test_within_bound_of_exact(self, fmt, N, K):
        x, wq = _case(fmt, N, K, N * 37 + K)
        y = (o.gemv_q4_0 if fmt == "q4_0" else o.gemv_q8_0)(x, wq, N, K)
        ref, mag = o.gemv_exact(fmt, x, wq, N, K)
        assert (np.abs(y.astype(np.float64) - ref) <= o.gemv_bound(K, mag)).all()

    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    def test_nonfinite_k0_n0(self, fmt):
        fn, qz = (o.gemv_q4_0, o.quantize_q4_0) if fmt == "q4_0" else (o.gemv_q8_0, o.quantize_q8_0)
        w = np.full((9, 64), 0.25, np.float32)
        for bad in (np.nan, np.inf, -np.inf):
            x = np.ones(64, np.float32)
            x[37] = bad
            assert np.isnan(fn(x, qz(w), 9, 64)).all()
        assert (fn(np.ones(0, np.float32), np.zeros(0, np.uint8), 5, 0) == 0).all()
        assert fn(np.ones(32, np.float32), np.zeros(0, np.uint8), 0, 32).shape == (0,)

    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    @pytest.mark.parametrize("N,K", SHAPES)
    def test_bitwise_equal_to_reference_scalar_table(self, ref_lib, fmt, N, K):
        x, wq = _case(fmt, N, K, N * 31 + K)
        y = (o.gemv_q4_0 if fmt == "q4_0" else o.gemv_q8_0)(x, wq, N, K)
        want = np.zeros(N, np.float32)
        fn = ref_lib.ref_gemv_q4_0 if fmt == "q4_0" else ref_lib.ref_gemv_q8_0
        assert fn(o.ISA["scalar"], N, K, x.ctypes.data_as(o._f32p), wq.ctypes.data_as(o._u8p),
                  want.ctypes.data_as(o._f32p)) == 0
        np.testing.assert_array_equal(y.view(np.uint32), want.view(np.uint32))

    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    def test_reference_simd_tables_within_bound(self, ref_lib, fmt):
        for isa in ("avx2", "avx512"):
            if not ref_lib.ref_table_available(o.ISA[isa]):
                continue
            for N, K in SHAPES:
                x, wq = _case(fmt, N, K, N + K)
                y = np.zeros(N, np.float32)
                fn = ref_lib.ref_gemv_q4_0 if fmt == "q4_0" else ref_lib.ref_gemv_q8_0
                fn(o.ISA[isa], N, K, x.ctypes.data_as(o._f32p), wq.ctypes.data_as(o._u8p),
                   y.ctypes.data_as(o._f32p))
                ref, mag = o.gemv_exact(fmt, x, wq, N, K)
                assert (np.abs(y.astype(np.float64) - ref) <= o.gemv_bound(K, mag)).all(), (isa, N, K)


class TestGemmTb:
    @pytest.mark.parametrize("fmt", ["fp32", "f16", "bf16"])
    @pytest.mark.parametrize("M,N,K", [(1, 37, 1), (1, 37, 17), (1, 4096, 300), (1, 64, 4099), (4, 33, 1027),
                                       (8, 45, 133)])
    def test_within_bound_and_equal_to_reference_scalar(self, ref_lib, fmt, M, N, K):
        rng = np.random.default_rng(M * 7 + N + K)
        A32, W32 = rng.standard_normal((M, K)).astype(np.float32), rng.standard_normal((N, K)).astype(np.float32)
        if fmt == "fp32":
            A, W, Ar, Wr = A32, W32, A32.astype(np.float64), W32.astype(np.float64)
        elif fmt == "f16":
            A, W = A32.astype(np.float16), W32.astype(np.float16)
            Ar, Wr = A.astype(np.float64), W.astype(np.float64)
        else:
            A, W = o.to_bf16_rne(A32), o.to_bf16_rne(W32)
            Ar, Wr = o.bf16_to_f32(A).astype(np.float64), o.bf16_to_f32(W).astype(np.float64)
        C = o.gemm_tb(fmt, A, W)
        bound = o.gemm_bound(K, np.abs(Ar) @ np.abs(Wr).T)
        assert (np.abs(C - Ar @ Wr.T) <= bound).all()
        want = np.zeros((M, N), np.float32)
        args = (o.ISA["scalar"], 1, M, N, K, 1.0, A.ctypes.data, K, W.ctypes.data, K, 0.0,
                want.ctypes.data_as(o._f32p), N)
        if fmt == "fp32":
            ref_lib.ref_sgemm(o.ISA["scalar"], 0, 1, M, N, K, 1.0, A.ctypes.data, K, W.ctypes.data, K, 0.0,
                              want.ctypes.data_as(o._f32p), N)
        else:
            (ref_lib.ref_sgemm_f16 if fmt == "f16" else ref_lib.ref_sgemm_bf16)(*args)
        np.testing.assert_array_equal(C.view(np.uint32), want.view(np.uint32))


class TestSilu:
    def test_bound_and_special_values(self):
        xs = np.concatenate([np.linspace(-200, 200, 20001, dtype=np.float32),
                             np.random.default_rng(1).uniform(-200, 200, 1000).astype(np.float32)])
        y = o.silu_scalar(xs)
        r = o.silu64(xs)
        assert (np.abs(y - r) <= 1e-35 + 1e-6 * np.abs(r)).all()
        s = o.silu_scalar(np.array([np.inf, -np.inf, np.nan, -1e30], np.float32))
        assert s[0] == np.inf and np.isnan(s[1]) and np.isnan(s[2]) and s[3] == 0

    def test_reference_avx2_silu_within_bound(self, ref_lib):
        if not ref_lib.ref_table_available(o.ISA["avx2"]):
            pytest.skip("no AVX2")
        xs = np.linspace(-200, 200, 20001, dtype=np.float32)
        y = np.zeros_like(xs)
        ref_lib.ref_silu(o.ISA["avx2"], xs.ctypes.data_as(o._f32p), y.ctypes.data_as(o._f32p), xs.size)
        r = o.silu64(xs)
        assert (np.abs(y - r) <= 1e-35 + 1e-6 * np.abs(r)).all()


# ─── planted mistakes: the checks above must catch them ────────────────────

class TestPlantedMistakes:
    """Each test plants a plausible mistake in a copy of the oracle (on the CPU)
    and shows that one of the pinning checks fails for it."""

    def test_swapped_nibble_order_fails_fixture(self):
        fx = np.load(FIXTURE, allow_pickle=False)
        good = o.q4_0_quantize_numpy(fx["w"]).reshape(20, 8, 18)
        bad = good.copy()
        bad[:, :, 2:] = (good[:, :, 2:] >> 4) | ((good[:, :, 2:] & 0x0F) << 4)
        assert not np.array_equal(bad.reshape(20, 144), fx["blocks"])

    def test_fused_multiply_add_quantizer_fails_fixture(self):
        """w*id + 8.5 in one rounding (float64 then cast) instead of two."""
        fx = np.load(FIXTURE, allow_pickle=False)
        w = fx["w"].reshape(-1, 8, 32).astype(np.float32)
        a = np.abs(w)
        first = np.take_along_axis(w, a.argmax(axis=2)[:, :, None], axis=2)[:, :, 0]
        d = (np.where(a.max(axis=2) > 0, first, 0).astype(np.float32) / np.float32(-8)).astype(np.float32)
        with np.errstate(divide="ignore", over="ignore"):
            idv = np.where(d != 0, np.float32(1) / d, 0).astype(np.float32)
        idv[np.isinf(idv)] = 0
        t = (w.astype(np.float64) * idv[:, :, None].astype(np.float64) + 8.5).astype(np.float32)
        q = np.minimum(np.trunc(t), 15).astype(np.uint8)
        assert not np.array_equal(q[:, :, :16] | (q[:, :, 16:] << 4), fx["blocks"].reshape(20, 8, 18)[:, :, 2:])

    def test_half_even_rounding_fails_q8_special_rows(self):
        w = q8_special_rows()
        good = o.q8_0_quantize_numpy(w)
        b = w.reshape(-1, 4, 32)
        d = (np.abs(b).max(axis=2) / np.float32(127)).astype(np.float32)
        with np.errstate(divide="ignore", over="ignore"):
            idv = np.where(d != 0, np.float32(1) / d, 0).astype(np.float32)
        idv[np.isinf(idv)] = 0
        q = np.round((b * idv[:, :, None]).astype(np.float32)).astype(np.int8)  # np.round: half to even
        assert not np.array_equal(q.view(np.uint8), good.reshape(-1, 4, 34)[:, :, 2:])

    def test_dropped_minus_eight_fails_bound(self):
        N, K = 33, 4096
        x, wq = _case("q4_0", N, K, 5)
        ref, mag = o.gemv_exact("q4_0", x, wq, N, K)
        dw, qw = o.q4_0_split(wq, N, K)
        qs, dx = o.quantize_x_q8(x)
        wrong = ((qw.astype(np.int64) + 8) * qs.reshape(1, -1, 32)).sum(axis=2) * dw * dx[None, :]
        assert not (np.abs(wrong.sum(axis=1) - ref) <= o.gemv_bound(K, mag)).all()

    def test_transposed_operand_fails_gemm_bound(self):
        rng = np.random.default_rng(0)
        A, W = rng.standard_normal((4, 33)).astype(np.float32), rng.standard_normal((33, 33)).astype(np.float32)
        C = o.gemm_tb("fp32", A, W.T.copy())  # W^T passed where W is expected
        bound = o.gemm_bound(33, np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64)).T)
        assert not (np.abs(C - A.astype(np.float64) @ W.astype(np.float64).T) <= bound).all()


class TestLlamaFormulas:
    """The numpy formulas of examples/llama/llama.py that the GPU kernels restate, pinned by
    numpy itself (the reduction model) and by float64 mathematics (norm, rotation, frequencies)."""

    @pytest.mark.parametrize("n", [1, 7, 8, 9, 100, 128, 129, 136, 260, 1000, 2048, 8191, 8192, 8193, 14336, 20000])
    def test_numpy_sum_model_equals_add_reduce(self, n):
        rng = np.random.default_rng(n)
        for s in (-3, 0, 3):
            q = (rng.standard_normal(n) * 10.0 ** s).astype(np.float32) ** 2
            got = o.numpy_sum_f32(q)
            assert got.view(np.uint32) == np.float32(np.add.reduce(q, dtype=np.float32)).view(np.uint32)

    def test_unchunked_pairwise_differs_above_8192(self):
        """A single pairwise tree over 14336 values is not numpy's sum (it reduces by 8192-chunks)."""
        rng = np.random.default_rng(0)
        differs = 0
        for _ in range(20):
            q = (rng.standard_normal(14336) * 30).astype(np.float32) ** 2
            differs += o.pairwise_sum_f32(q).view(np.uint32) != np.float32(np.add.reduce(q)).view(np.uint32)
        assert differs > 0

    def test_rms_norm_close_to_float64(self):
        rng = np.random.default_rng(1)
        for n in (64, 2048, 14336):
            x = rng.standard_normal(n).astype(np.float32) * np.float32(7)
            w = rng.standard_normal(n).astype(np.float32)
            y, y64 = o.rms_norm(x, w, 1e-5), o.rms_norm64(x, w, 1e-5)
            # var: sum error <= log2(n) u, division/scale/products a few more roundings.
            assert (np.abs(y - y64) <= (math.log2(n) + 8) * 2.0 ** -24 * np.abs(y64) + 1e-30).all()

    def test_rms_norm_planted_float32_scale_fails(self):
        """Computing 1/sqrt(var + eps) in float32 (instead of float64) changes some outputs."""
        rng = np.random.default_rng(2)
        changed = 0
        for _ in range(50):
            x = rng.standard_normal(2048).astype(np.float32)
            w = np.ones(2048, np.float32)
            var = np.mean(x * x, dtype=np.float32)
            wrong = w * (x * (np.float32(1) / np.sqrt(var + np.float32(1e-5))))
            changed += not np.array_equal(wrong, o.rms_norm(x, w, 1e-5))
        assert changed > 0

    @pytest.mark.parametrize("interleaved", [True, False])
    def test_rope_is_a_rotation(self, interleaved):
        rng = np.random.default_rng(3)
        hd = 64
        inv = o.rope_inv_freq(hd, 500000.0, None)
        pos = 123
        cos, sin = o.rope_cos_sin(inv, pos)
        x = rng.standard_normal((8, hd)).astype(np.float32)
        y = o.rope(x, cos, sin, interleaved).astype(np.float64)
        ang = pos * inv.astype(np.float64)
        if interleaved:
            z = (x[:, 0::2] + 1j * x[:, 1::2]).astype(np.complex128) * np.exp(1j * ang)
            ref = np.empty((8, hd))
            ref[:, 0::2], ref[:, 1::2] = z.real, z.imag
        else:
            z = (x[:, :hd // 2] + 1j * x[:, hd // 2:]).astype(np.complex128) * np.exp(1j * ang)
            ref = np.concatenate([z.real, z.imag], axis=1)
        assert np.abs(y - ref).max() < 1e-4  # angles are float32 (pos * inv_freq rounded), as in the example
        np.testing.assert_allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x.astype(np.float64), axis=1), rtol=1e-6)

    def test_rope_planted_swapped_sign_fails(self):
        rng = np.random.default_rng(4)
        cos, sin = o.rope_cos_sin(o.rope_inv_freq(64, 500000.0, None), 5)
        x = rng.standard_normal((2, 64)).astype(np.float32)
        good = o.rope(x, cos, sin, True)
        a, b = x[:, 0::2], x[:, 1::2]
        bad = np.empty_like(x)
        bad[:, 0::2], bad[:, 1::2] = a * cos[:32] + b * sin[:32], b * cos[:32] - a * sin[:32]
        assert not np.allclose(good, bad)

    def test_rope_inv_freq_default_and_llama3(self):
        hd, theta = 64, 500000.0
        base = o.rope_inv_freq(hd, theta, None).astype(np.float64)
        np.testing.assert_allclose(base, theta ** (-np.arange(0, hd, 2) / hd), rtol=2e-6)
        rs = {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
              "original_max_position_embeddings": 8192}
        sc = o.rope_inv_freq(hd, theta, rs).astype(np.float64)
        wl = 2 * math.pi / base
        hi = wl < 8192 / 4.0
        lo = wl > 8192 / 1.0
        np.testing.assert_allclose(sc[hi], base[hi], rtol=1e-6)       # short wavelengths kept
        np.testing.assert_allclose(sc[lo], base[lo] / 32.0, rtol=1e-6)  # long ones divided by factor
        mid = ~hi & ~lo
        s = (8192 / wl[mid] - 1.0) / 3.0
        np.testing.assert_allclose(sc[mid], (1 - s) * base[mid] / 32.0 + s * base[mid], rtol=1e-5)


class TestReferenceSimdOrder:
    """The oracle's restatements of the reference's SIMD-table arithmetic orders, pinned bit for
    bit to the reference's own build (its widest table on this CPU: AVX-512 here; the Q4_0 loop,
    SiLU and softmax are shared with the AVX2 table)."""

    @pytest.fixture
    def simd(self, ref_lib):
        isa = o.ref_best_isa()
        if isa not in ("avx2", "avx512"):
            pytest.skip("the reference's SIMD tables need AVX2")
        return ref_lib, o.ISA[isa]

    @pytest.mark.parametrize("N,K", [(1, 32), (2, 64), (3, 64), (7, 96), (9, 2048), (17, 4096), (33, 11008),
                                     (1001, 2048), (2048, 8192)])
    def test_gemv_q4_0(self, simd, N, K):
        R, isa = simd
        rng = np.random.default_rng(N + K)
        wq = o.quantize_q4_0((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
        x = (rng.standard_normal(K) * 3).astype(np.float32)
        yr = np.empty(N, np.float32)
        R.ref_gemv_q4_0(isa, N, K, x.ctypes.data_as(o._f32p), wq.ctypes.data_as(o._u8p), yr.ctypes.data_as(o._f32p))
        np.testing.assert_array_equal(o.gemv_q4_0_simd(x, wq, N, K).view(np.uint32), yr.view(np.uint32))

    def test_scalar_order_differs(self, simd):
        """The scalar table's sequential sum is a different function: a planted-order check."""
        R, isa = simd
        rng = np.random.default_rng(1)
        wq = o.quantize_q4_0((rng.standard_normal((512, 2048)) * 0.02).astype(np.float32))
        x = rng.standard_normal(2048).astype(np.float32)
        assert not np.array_equal(o.gemv_q4_0(x, wq, 512, 2048), o.gemv_q4_0_simd(x, wq, 512, 2048))

    @pytest.mark.parametrize("M,N,K", [(4, 1, 64), (4, 160, 64), (1, 5, 100), (3, 7, 31), (8, 9, 200)])
    def test_sgemm_trans_b_few_rows(self, simd, M, N, K):
        R, isa = simd
        rng = np.random.default_rng(M * N * K)
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.standard_normal((N, K)).astype(np.float32)
        Cr = np.zeros((M, N), np.float32)
        R.ref_sgemm(isa, 0, 1, M, N, K, 0.125, A.ctypes.data, K, B.ctypes.data, K, 0.0, Cr.ctypes.data_as(o._f32p), N)
        np.testing.assert_array_equal(o.sgemm_tb_simd(A, B, 0.125).view(np.uint32), Cr.view(np.uint32))

    @pytest.mark.parametrize("M,N,K", [(4, 64, 1), (4, 64, 37), (4, 64, 160), (3, 64, 100)])
    def test_sgemm_direct(self, simd, M, N, K):
        R, isa = simd
        rng = np.random.default_rng(M + N + K)
        A = np.abs(rng.standard_normal((M, K))).astype(np.float32)
        B = rng.standard_normal((K, N)).astype(np.float32)
        Cr = np.zeros((M, N), np.float32)
        R.ref_sgemm(isa, 0, 0, M, N, K, 1.0, A.ctypes.data, K, B.ctypes.data, N, 0.0, Cr.ctypes.data_as(o._f32p), N)
        np.testing.assert_array_equal(o.sgemm_nn_simd(A, B).view(np.uint32), Cr.view(np.uint32))

    def test_silu(self, simd):
        R, isa = simd
        rng = np.random.default_rng(2)
        x = np.concatenate([rng.standard_normal(100000) * 10, rng.uniform(-100, 100, 100000),
                            np.array([0, -0.0, 88, -88, 88.5, -88.5, 1e30, -1e30, np.inf, -np.inf])]).astype(np.float32)
        yr = np.empty_like(x)
        R.ref_silu(isa, x.ctypes.data_as(o._f32p), yr.ctypes.data_as(o._f32p), x.size)
        np.testing.assert_array_equal(o.silu_simd(x).view(np.uint32), yr.view(np.uint32))

    def test_softmax(self, simd):
        R, isa = simd
        rng = np.random.default_rng(3)
        for n in list(range(1, 40)) + [100, 127, 128, 129, 160, 1000]:
            s = (rng.standard_normal(n) * rng.uniform(0.1, 20)).astype(np.float32)
            r = np.empty_like(s)
            R.ref_softmax_row(isa, s.ctypes.data_as(o._f32p), r.ctypes.data_as(o._f32p), n)
            np.testing.assert_array_equal(o.softmax_simd(s).view(np.uint32), r.view(np.uint32), err_msg=str(n))

    def test_fast_exp_accuracy(self):
        """The restated exp against float64 (simd_math.hpp:57: absolute error <= 1.22e-7 on
        [-87.3, 88.4] relative to values of order 1)."""
        z = np.linspace(-10, 10, 20001).astype(np.float32)
        got = np.array([o.lib().smko_fast_exp(float(v)) for v in z[::50]])
        ref = np.exp(z[::50].astype(np.float64))
        assert (np.abs(got - ref) / np.maximum(ref, 1) <= 2.5e-7).all()
