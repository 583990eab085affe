"""GPU parity of the quantized decode path against the CPU oracle (oracle/), through the C ABI.

Bars (the reference's own, q4_0.hpp:25-30, q8_0.hpp:18-28):
  * x's Q8 quants and FP32 scales: bit-exact;
  * every per-block int32 sum: bit-exact;
  * weight quantizers: byte-exact (llama.cpp fixture, special blocks, random);
  * y: |y - y64| <= 2*(K/32 + 4)*2^-24 * sum_b |dw dx| sum_i |qw qx| against the float64
    exact sum of the same quantized operands; non-finite x -> all NaN; K = 0 -> zeros.
At the BASELINE shapes (8192x2048, 2048x8192, 14336x4096, 128256x4096) the same bound is
checked in full, plus a checksum-of-checksums property on the rotated copies of the bench.
"""

import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as o
from tests import gpu_util as g

pytestmark = pytest.mark.gpu

BB = {"q4_0": 18, "q8_0": 34}
QUANT = {"q4_0": o.quantize_q4_0, "q8_0": o.quantize_q8_0}
SHAPES = [(1, 32), (7, 64), (8, 96), (9, 128), (13, 160), (17, 352), (100, 4096), (33, 11008), (64, 2048),
          (300, 2048), (1, 14336), (5, 8192)]


def _inputs(fmt, N, K, seed, xscale=4.0):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((N, K)).astype(np.float32)
    x = (rng.standard_normal(K) * xscale).astype(np.float32)
    return x, QUANT[fmt](w)


def d_gemv(fmt, x, wq, N, K, offset=0):
    """y from smk_d_gemv_<fmt> on device copies; Wq placed `offset` bytes into its buffer."""
    xd = g.dev(x)
    staged = np.full(wq.nbytes + offset + 16, 0xEE, np.uint8)
    staged[offset:offset + wq.nbytes] = wq.reshape(-1)
    wbuf = g.dev(staged)
    yd = g.empty(4 * N + 64)
    g.call(f"smk_d_gemv_{fmt}", N, K, g.ptr(xd), g.ptr(wbuf, offset), g.ptr(yd), g.stream())
    out = g.host(yd, np.float32)
    assert (out[N:N + 16].view(np.uint32) == 0xEEEEEEEE).all(), "wrote past y[N)"
    return out[:N]


class TestXQuant:
    @pytest.mark.parametrize("K", [32, 96, 2048, 4096, 14336])
    def test_bit_exact(self, K):
        x = (np.random.default_rng(K).standard_normal(K) * 3).astype(np.float32)
        x[:32] = np.arange(-16, 16) + 0.5          # exact ties at d = 1? (amax 15.5): round half away
        if K >= 96:
            x[32:64] = 0.0                          # zero block
            x[64:96] = np.float32(1e-39) * np.sign(np.random.default_rng(1).standard_normal(32)).astype(np.float32)
        qs_ref, dx_ref = o.quantize_x_q8(x)
        xd, qd, dd, bad = g.dev(x), g.empty(K), g.empty(4 * (K // 32)), g.empty(4, 0)
        g.call("smk_d_quantize_x_q8", K, g.ptr(xd), g.ptr(qd), g.ptr(dd), g.ptr(bad), g.stream())
        np.testing.assert_array_equal(g.host(qd, np.int8, K), qs_ref)
        np.testing.assert_array_equal(g.host(dd, np.uint32, K // 32), dx_ref.view(np.uint32))
        assert g.host(bad, np.int32)[0] == 0

    def test_division_free_scale_and_rounding_exhaustive(self):
        """The quantizer's division-free d = amax/127, id = 1/d and roundf (device_common.hpp
        q8_scale, round_half_away) equal the IEEE forms for every finite amax >= 0 and every
        |p| <= 127.5, checked on the device itself (smk_selfcheck_q8)."""
        out = (ctypes.c_uint * 2)()
        g.call("smk_selfcheck_q8", ctypes.addressof(out))
        assert (out[0], out[1]) == (0, 0), f"scale mismatches {out[0]}, rounding mismatches {out[1]}"

    def test_nonfinite_flag(self):
        x = np.ones(256, np.float32)
        x[77] = np.inf
        xd, qd, dd, bad = g.dev(x), g.empty(256), g.empty(32), g.empty(4, 0)
        g.call("smk_d_quantize_x_q8", 256, g.ptr(xd), g.ptr(qd), g.ptr(dd), g.ptr(bad), g.stream())
        assert g.host(bad, np.int32)[0] == 1


class TestBlockSums:
    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    @pytest.mark.parametrize("N,K", [(7, 64), (33, 4096), (17, 352)])
    def test_bit_exact(self, fmt, N, K):
        x, wq = _inputs(fmt, N, K, N + K)
        qs, _ = o.quantize_x_q8(x)
        want = o.block_sums(fmt, qs, wq, N, K)
        qd, wd, out = g.dev(qs), g.dev(wq), g.empty(4 * N * (K // 32))
        g.call("smk_d_block_sums", BB[fmt], N, K, g.ptr(qd), g.ptr(wd), g.ptr(out), g.stream())
        np.testing.assert_array_equal(g.host(out, np.int32, N * (K // 32)).reshape(N, -1), want)


class TestQuantizeWeights:
    def _run(self, fmt, w):
        w = np.ascontiguousarray(w, np.float32)
        rows, K = w.reshape(-1, w.shape[-1]).shape
        out_bytes = rows * (K // 32) * BB[fmt]
        wd, od, bad = g.dev(w), g.empty(out_bytes), g.empty(4, 0)
        g.call("smk_d_quantize", BB[fmt], rows, K, g.ptr(wd), g.ptr(od), g.ptr(bad), g.stream())
        return g.host(od, np.uint8, out_bytes), g.host(bad, np.int32)[0]

    def test_q4_0_llama_cpp_fixture(self):
        fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "q4_0_ggml_v0.7.0.npz"), allow_pickle=False)
        got, bad = self._run("q4_0", fx["w"])
        assert bad == 0
        np.testing.assert_array_equal(got.reshape(fx["blocks"].shape), fx["blocks"])

    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    def test_random_and_special(self, fmt):
        from tests.test_oracle import q8_special_rows
        rng = np.random.default_rng(9)
        special = q8_special_rows()[:, :128].repeat(2, axis=1)
        if fmt == "q4_0":
            special = special[[0, 1, 3, 4, 5]]  # row 2's scales overflow Q4_0's float16 scale
        w = np.concatenate([rng.standard_normal((64, 256)).astype(np.float32) * 3, special])
        w[0, :32] = np.where(np.arange(32) % 2, 1e-44, -1e-44).astype(np.float32)
        w[1, :32] = 1.0
        w[2, :32] = -0.0
        got, bad = self._run(fmt, w)
        assert bad == 0
        np.testing.assert_array_equal(got.reshape(w.shape[0], -1), QUANT[fmt](w))

    @pytest.mark.parametrize("fmt,limit", [("q4_0", 8 * 65520.0), ("q8_0", 127 * 65520.0)])
    def test_rejections(self, fmt, limit):
        for bad_v in (np.nan, np.inf, limit):
            w = np.ones((3, 64), np.float32)
            w[1, 40] = bad_v
            assert self._run(fmt, w)[1] == 1
        w = np.ones((3, 64), np.float32)
        w[1, 40] = limit * 65504.0 / 65520.0
        assert self._run(fmt, w)[1] == 0


class TestGemv:
    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    @pytest.mark.parametrize("N,K", SHAPES)
    def test_within_bound(self, fmt, N, K):
        x, wq = _inputs(fmt, N, K, N * 37 + K)
        y = d_gemv(fmt, x, wq, N, K)
        ref, mag = o.gemv_exact(fmt, x, wq, N, K)
        err = np.abs(y.astype(np.float64) - ref)
        assert (err <= o.gemv_bound(K, mag)).all(), f"max err/bound {np.max(err / o.gemv_bound(K, mag)):.3g}"

    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    def test_extreme_quants(self, fmt):
        N, K = 9, 4096
        rng = np.random.default_rng(3)
        w = np.where(rng.random((N, K)) < 0.5, -1.0, 1.0).astype(np.float32) * 1000.0
        x = np.where(rng.random(K) < 0.5, -1.0, 1.0).astype(np.float32) * 1e3
        wq = QUANT[fmt](w)
        y = d_gemv(fmt, x, wq, N, K)
        ref, mag = o.gemv_exact(fmt, x, wq, N, K)
        assert (np.abs(y - ref) <= o.gemv_bound(K, mag)).all()

    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    def test_nan_k0_n0(self, fmt):
        w = np.full((9, 64), 0.25, np.float32)
        for bad in (np.nan, np.inf, -np.inf):
            x = np.ones(64, np.float32)
            x[37] = bad
            assert np.isnan(d_gemv(fmt, x, QUANT[fmt](w), 9, 64)).all()
        assert (d_gemv(fmt, np.ones(0, np.float32), np.zeros(0, np.uint8), 5, 0) == 0).all()
        yd = g.empty(64)
        g.call(f"smk_d_gemv_{fmt}", 0, 32, 0, 0, g.ptr(yd), g.stream())
        assert (g.host(yd, np.uint8) == 0xEE).all()

    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    def test_two_byte_offset_takes_generic_path(self, fmt):
        N, K = 13, 2048
        x, wq = _inputs(fmt, N, K, 4)
        a = d_gemv(fmt, x, wq, N, K)
        b = d_gemv(fmt, x, wq, N, K, offset=2)
        ref, mag = o.gemv_exact(fmt, x, wq, N, K)
        assert (np.abs(b - ref) <= o.gemv_bound(K, mag)).all()
        assert (np.abs(a - ref) <= o.gemv_bound(K, mag)).all()

    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    @pytest.mark.parametrize("lpr", [8, 16, 32, 64])
    def test_every_lane_split(self, fmt, lpr):
        N, K = 77, 4096
        x, wq = _inputs(fmt, N, K, lpr)
        g.call("smk_set_gemv_tuning", lpr, 0, 0, 0)
        try:
            y = d_gemv(fmt, x, wq, N, K)
        finally:
            g.call("smk_set_gemv_tuning", 0, 0, 0, 0)
        ref, mag = o.gemv_exact(fmt, x, wq, N, K)
        assert (np.abs(y - ref) <= o.gemv_bound(K, mag)).all()


class TestQ4ReferenceOrder:
    """Q4_0 y is bit-exact with the reference's SIMD tables (q4_0_rows.hpp: four FMA chains per
    row, the odd last row in eight), restated in oracle/smk_oracle.c and pinned there to the
    reference's own AVX-512 build; against oracle/_ref directly where it is present."""

    SHAPES = [(1, 64), (2, 64), (3, 64), (7, 96), (8, 2048), (9, 2048), (77, 4096), (33, 11008), (300, 2048),
              (1001, 2048), (5, 8192), (3072, 2048), (2048, 8192), (4, 14336)]

    @pytest.mark.parametrize("N,K", SHAPES)
    def test_bit_exact_with_reference_order(self, N, K):
        x, wq = _inputs("q4_0", N, K, N * 31 + K)
        y = d_gemv("q4_0", x, wq, N, K)
        np.testing.assert_array_equal(y.view(np.uint32), o.gemv_q4_0_simd(x, wq, N, K).view(np.uint32))
        R = o.ref()
        if R is not None and o.ref_best_isa() in ("avx2", "avx512"):
            yr = np.empty(N, np.float32)
            R.ref_gemv_q4_0(o.ISA[o.ref_best_isa()], N, K, x.ctypes.data_as(o._f32p), wq.ctypes.data_as(o._u8p),
                            yr.ctypes.data_as(o._f32p))
            np.testing.assert_array_equal(y.view(np.uint32), yr.view(np.uint32))

    @pytest.mark.parametrize("N,K", [(13, 2048), (12, 96), (5, 32)])
    def test_generic_path_same_order(self, N, K):
        """Odd K/32 and a 2-byte aligned W take the generic kernel: same bits."""
        x, wq = _inputs("q4_0", N, K, 99)
        ref = o.gemv_q4_0_simd(x, wq, N, K)
        for off in (0, 2):
            y = d_gemv("q4_0", x, wq, N, K, offset=off)
            np.testing.assert_array_equal(y.view(np.uint32), ref.view(np.uint32))

    @pytest.mark.parametrize("mode", [0, 1, 2])
    def test_every_weight_load_form_same_bits(self, mode):
        """Pair loads, and weights streamed through LDS one or two groups of rows ahead
        (smk_set_q4_stream): y bit-exact with the reference order in each form, at the decode
        shapes, config 1, a Llama-3-8B shape and uneven workgroups."""
        g.call("smk_set_q4_stream", mode)
        g.call("smk_set_q4_tiles", -1)  # the row-group kernel, whose load forms these are
        try:
            for N, K in ((8192, 2048), (3072, 2048), (16384, 2048), (2048, 8192), (1000, 4096), (14336, 4096)):
                x, wq = _inputs("q4_0", N, K, 7 * N + K + mode)
                y = d_gemv("q4_0", x, wq, N, K)
                np.testing.assert_array_equal(y.view(np.uint32), o.gemv_q4_0_simd(x, wq, N, K).view(np.uint32),
                                              err_msg=f"mode {mode} N={N} K={K}")
        finally:
            g.call("smk_set_q4_stream", -1)
            g.call("smk_set_q4_tiles", 0)

    # K-chunk tiles: full chunks (K % 2048 == 0), a partial last chunk (K/32 % 64 != 0), one
    # partial chunk only (K = 256, 768), long rows (14336, 32768), uneven workgroups, and the
    # Llama-3-8B / BASELINE shapes.
    TILED = [(8192, 2048), (14336, 4096), (4096, 14336), (2048, 8192), (1000, 4096), (513, 2304), (40, 256),
             (17, 768), (250, 11008), (64, 32768), (4098, 4096), (1, 4096), (31, 2048)]

    @pytest.mark.parametrize("tiles", [2, 3, 4])
    def test_tiled_kernel_every_depth_same_bits(self, tiles):
        """The K-chunk tiled kernel (smk_set_q4_tiles), 2, 3 and 4 tiles in flight: y bit-exact
        with the reference order at every shape of TILED (and so with the row-group kernel)."""
        g.call("smk_set_q4_tiles", tiles)
        try:
            for N, K in self.TILED:
                x, wq = _inputs("q4_0", N, K, 3 * N + K + tiles)
                y = d_gemv("q4_0", x, wq, N, K)
                np.testing.assert_array_equal(y.view(np.uint32), o.gemv_q4_0_simd(x, wq, N, K).view(np.uint32),
                                              err_msg=f"tiles {tiles} N={N} K={K}")
        finally:
            g.call("smk_set_q4_tiles", 0)

    def test_tiled_kernel_nonfinite_x_and_extremes(self):
        """A NaN in x makes every y NaN; saturated quants (|x| at a block's max, nibbles 0 and 15)
        keep the exact integer dots at their extremes; the tiled kernel against the reference order."""
        N, K = 300, 4096
        x, wq = _inputs("q4_0", N, K, 17)
        wq = wq.copy()
        blk = wq.reshape(N, K // 32, 18)
        blk[::3, :, 2:] = 0xFF      # q = 15 everywhere
        blk[1::3, :, 2:] = 0x00     # q = 0 everywhere
        x[:32] = 127.0
        x[32:64] = -127.0
        y = d_gemv("q4_0", x, wq, N, K)
        np.testing.assert_array_equal(y.view(np.uint32), o.gemv_q4_0_simd(x, wq, N, K).view(np.uint32))
        x[4000] = np.nan
        y = d_gemv("q4_0", x, wq, N, K)
        assert np.isnan(y).all()

    @pytest.mark.parametrize("lpr", [8, 16, 32, 64])
    def test_lane_split_does_not_change_bits(self, lpr):
        N, K = 131, 4096
        x, wq = _inputs("q4_0", N, K, 5)
        g.call("smk_set_gemv_tuning", lpr, 0, 0, 0)
        try:
            y = d_gemv("q4_0", x, wq, N, K)
        finally:
            g.call("smk_set_gemv_tuning", 0, 0, 0, 0)
        np.testing.assert_array_equal(y.view(np.uint32), o.gemv_q4_0_simd(x, wq, N, K).view(np.uint32))

    def test_config_1_shape(self):
        x, w = o.synthetic(0, [(2048,), (8192, 2048)], [1.0, 0.02])
        wq = o.quantize_q4_0(w)
        y = d_gemv("q4_0", x, wq, 8192, 2048)
        np.testing.assert_array_equal(y.view(np.uint32), o.gemv_q4_0_simd(x, wq, 8192, 2048).view(np.uint32))


class TestBatched:
    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    @pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
    def test_rows_equal_gemv_bitwise(self, fmt, M):
        N, K = 96, 4096
        rng = np.random.default_rng(M)
        X = rng.standard_normal((M, K)).astype(np.float32)
        X[M - 1, 5] = np.nan if M > 1 else X[M - 1, 5]   # one non-finite row: only that row is NaN
        wq = QUANT[fmt](rng.standard_normal((N, K)).astype(np.float32))
        xd, wd, yd = g.dev(X), g.dev(wq), g.empty(4 * M * N)
        g.call(f"smk_d_gemm_{fmt}", M, N, K, g.ptr(xd), K, g.ptr(wd), g.ptr(yd), N, g.stream())
        Y = g.host(yd, np.float32, M * N).reshape(M, N)
        for m in range(M):
            y1 = d_gemv(fmt, X[m], wq, N, K)
            np.testing.assert_array_equal(Y[m].view(np.uint32), y1.view(np.uint32))


def d_gemm(fmt, X, wq, N, K, offset=0):
    """Y [M, N] from smk_d_gemm_<fmt> on device copies (Wq `offset` bytes into its buffer); the
    4 KiB after Y must stay untouched."""
    M = X.shape[0]
    staged = np.full(wq.nbytes + offset + 16, 0xEE, np.uint8)
    staged[offset:offset + wq.nbytes] = wq.reshape(-1)
    xd, wd, yd = g.dev(X), g.dev(staged), g.dev(np.full(M * N + 1024, 0xEEEEEEEE, np.uint32))
    g.call(f"smk_d_gemm_{fmt}", M, N, K, g.ptr(xd), K, g.ptr(wd, offset), g.ptr(yd), N, g.stream())
    out = g.host(yd, np.uint32, M * N + 1024)
    assert (out[M * N:] == 0xEEEEEEEE).all(), "wrote past Y"
    return out[:M * N].view(np.float32).reshape(M, N)


class TestBatchedMatrixCores:
    """Q4_0 with several rows of x runs on the int8 matrix cores (gemm_q4_mfma.hip); every row must
    equal the reference's SIMD order for that row (oracle/smk_oracle.c, pinned to the reference's
    AVX-512 build) bit for bit -- the exact integer block sums, the four FMA chains per output and
    the final (a0 + a2) + (a1 + a3)."""

    # (M, N, K, W byte offset): K % 1024 == 0 with a 16-byte aligned W takes the streaming kernel,
    # the rest (K % 64 == 0, W 4-byte aligned) the whole-image kernel; odd N ends in the one-row
    # kernels; one launch holds 4, 8, 16 or 32 rows of x.
    CASES = [(2, 96, 4096, 0), (3, 64, 2048, 0), (4, 130, 64, 0), (5, 48, 128, 0), (8, 96, 4096, 0),
             (9, 32, 2048, 0), (16, 64, 4096, 0), (17, 80, 1024, 0), (31, 16, 2048, 0), (32, 200, 4096, 0),
             (33, 50, 4096, 0), (64, 34, 2048, 0), (12, 40, 14336, 0), (20, 18, 8192, 0), (7, 97, 2048, 0),
             (32, 1, 4096, 0), (6, 64, 2048, 4), (32, 48, 1088, 0), (13, 36, 4096, 4)]

    @pytest.fixture(autouse=True)
    def _matrix_cores_from_two_rows(self):
        g.call("smk_set_q4_mfma_min_rows", 2)
        yield
        g.call("smk_set_q4_mfma_min_rows", 0)

    @pytest.mark.parametrize("M,N,K,off", CASES)
    def test_rows_bit_exact_with_reference_order(self, M, N, K, off):
        rng = np.random.default_rng(M * 1000 + N + K)
        X = (rng.standard_normal((M, K)) * 2).astype(np.float32)
        wq = o.quantize_q4_0((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
        Y = d_gemm("q4_0", X, wq, N, K, offset=off)
        for m in range(M):
            ref = o.gemv_q4_0_simd(X[m], wq, N, K)
            np.testing.assert_array_equal(Y[m].view(np.uint32), ref.view(np.uint32), err_msg=f"row {m}")

    @pytest.mark.parametrize("M", [2, 4, 8, 32])
    def test_equals_eight_row_gemv_path(self, M):
        """The matrix-core path, the 8-row GEMV launches and the built-in switch give the same bits."""
        N, K = 256, 4096
        rng = np.random.default_rng(M)
        X = rng.standard_normal((M, K)).astype(np.float32)
        wq = o.quantize_q4_0(rng.standard_normal((N, K)).astype(np.float32))
        Y = d_gemm("q4_0", X, wq, N, K)
        g.call("smk_set_q4_mfma_min_rows", 1 << 30)
        Y8 = d_gemm("q4_0", X, wq, N, K)
        g.call("smk_set_q4_mfma_min_rows", 0)
        Yd = d_gemm("q4_0", X, wq, N, K)
        np.testing.assert_array_equal(Y.view(np.uint32), Y8.view(np.uint32))
        np.testing.assert_array_equal(Y.view(np.uint32), Yd.view(np.uint32))

    def test_nonfinite_rows_and_extremes(self):
        """A row of x with a NaN or an infinity is NaN, the others exact; saturated quants
        (x blocks at +-amax, weight nibbles 0 and 15) stay exact."""
        M, N, K = 12, 64, 2048
        rng = np.random.default_rng(4)
        X = rng.standard_normal((M, K)).astype(np.float32)
        X[3, 100] = np.nan
        X[7, 2047] = -np.inf
        X[9] = np.where(rng.standard_normal(K) > 0, 1.0, -1.0).astype(np.float32) * 1e30
        X[10] = 0.0
        w = rng.standard_normal((N, K)).astype(np.float32)
        w[::2] = np.where(w[::2] > 0, 1.0, -1.0) * np.abs(w[::2]).max()
        wq = o.quantize_q4_0(w)
        Y = d_gemm("q4_0", X, wq, N, K)
        for m in range(M):
            ref = o.gemv_q4_0_simd(X[m], wq, N, K)
            if m in (3, 7):
                assert np.isnan(Y[m]).all() and np.isnan(ref).all()
            else:
                np.testing.assert_array_equal(Y[m].view(np.uint32), ref.view(np.uint32), err_msg=f"row {m}")

    @pytest.mark.parametrize("M", [3, 4, 8])
    def test_nonfinite_rows_in_kernel_quantizer(self, M):
        """A launch of 4 or 8 rows of x (the streaming kernel's smallest images): a row with a NaN
        or an infinity is NaN; saturated and zero rows stay exact."""
        N, K = 64, 2048
        rng = np.random.default_rng(40 + M)
        X = rng.standard_normal((M, K)).astype(np.float32)
        X[0, 1000] = np.nan
        X[M - 1, 5] = np.inf
        X[1] = np.where(rng.standard_normal(K) > 0, 1.0, -1.0).astype(np.float32) * 1e30
        if M > 3:
            X[2] = 0.0
        wq = o.quantize_q4_0(rng.standard_normal((N, K)).astype(np.float32))
        Y = d_gemm("q4_0", X, wq, N, K)
        for m in range(M):
            ref = o.gemv_q4_0_simd(X[m], wq, N, K)
            if m in (0, M - 1):
                assert np.isnan(Y[m]).all() and np.isnan(ref).all()
            else:
                np.testing.assert_array_equal(Y[m].view(np.uint32), ref.view(np.uint32), err_msg=f"row {m}")

    @pytest.mark.parametrize("M,ldx,xoff", [(4, 2049, 0), (8, 2048, 1), (8, 2052, 0), (5, 4100, 0)])
    def test_row_stride_and_alignment_of_x(self, M, ldx, xoff):
        """x rows at any stride (odd, padded) and any 4-byte alignment: every row equals the
        reference order's."""
        N, K = 96, 2048 if ldx < 4096 else 4096
        rng = np.random.default_rng(ldx + xoff)
        buf = rng.standard_normal(xoff + M * ldx).astype(np.float32)
        X = np.stack([buf[xoff + m * ldx:xoff + m * ldx + K] for m in range(M)])
        wq = o.quantize_q4_0(rng.standard_normal((N, K)).astype(np.float32))
        xd, wd, yd = g.dev(buf), g.dev(wq), g.empty(4 * M * N)
        g.call("smk_d_gemm_q4_0", M, N, K, g.ptr(xd, 4 * xoff), ldx, g.ptr(wd), g.ptr(yd), N, g.stream())
        Y = g.host(yd, np.float32, M * N).reshape(M, N)
        for m in range(M):
            ref = o.gemv_q4_0_simd(X[m], wq, N, K)
            np.testing.assert_array_equal(Y[m].view(np.uint32), ref.view(np.uint32), err_msg=f"row {m}")

    def test_two_byte_aligned_w_takes_gemv_path(self):
        M, N, K = 6, 40, 2048
        rng = np.random.default_rng(6)
        X = rng.standard_normal((M, K)).astype(np.float32)
        wq = o.quantize_q4_0(rng.standard_normal((N, K)).astype(np.float32))
        Y = d_gemm("q4_0", X, wq, N, K, offset=2)
        for m in range(M):
            np.testing.assert_array_equal(Y[m].view(np.uint32), o.gemv_q4_0_simd(X[m], wq, N, K).view(np.uint32))

    def test_config_4_shape(self):
        """BASELINE config 4 at M = 32: N = 14336, K = 4096, x ~ N(0,1), W ~ N(0,0.02); every row
        against the one-row device GEMV (itself bit-exact with the reference order), eight rows
        against the oracle."""
        M, N, K = 32, 14336, 4096
        X, w = o.synthetic(4, [(M, K), (N, K)], [1.0, 0.02])
        wq = o.quantize_q4_0(w)
        del w
        Y = d_gemm("q4_0", X, wq, N, K)
        for m in range(M):
            np.testing.assert_array_equal(Y[m].view(np.uint32), d_gemv("q4_0", X[m], wq, N, K).view(np.uint32))
        for m in (0, 5, 17, 31):
            np.testing.assert_array_equal(Y[m].view(np.uint32), o.gemv_q4_0_simd(X[m], wq, N, K).view(np.uint32))

    def test_q8_0_more_than_eight_rows(self):
        M, N, K = 13, 70, 2048
        rng = np.random.default_rng(13)
        X = rng.standard_normal((M, K)).astype(np.float32)
        wq = o.quantize_q8_0(rng.standard_normal((N, K)).astype(np.float32))
        Y = d_gemm("q8_0", X, wq, N, K)
        for m in range(M):
            np.testing.assert_array_equal(Y[m].view(np.uint32), d_gemv("q8_0", X[m], wq, N, K).view(np.uint32))


class TestBaselineShapes:
    """Full BASELINE.json configurations, checked against the exact float64 sum."""

    @pytest.mark.parametrize("fmt,N,K,seed", [("q4_0", 8192, 2048, 0), ("q8_0", 8192, 2048, 1),
                                              ("q8_0", 2048, 8192, 1), ("q4_0", 14336, 4096, 3)])
    def test_config_shapes(self, fmt, N, K, seed):
        x, w = o.synthetic(seed, [(K,), (N, K)], [1.0, 0.02])
        wq = QUANT[fmt](w)
        y = d_gemv(fmt, x, wq, N, K)
        ref, mag = o.gemv_exact(fmt, x, wq, N, K)
        assert (np.abs(y - ref) <= o.gemv_bound(K, mag)).all()

    def test_lm_head_rows_and_checksum(self):
        """Q4_0 lm_head 128256x4096: rows compared in slices; the sum over all outputs equals the
        float64 exact sum within the summed bound (a checksum of checksums)."""
        N, K = 128256, 4096
        x, w = o.synthetic(3, [(K,), (N, K)], [1.0, 0.02])
        wq = QUANT["q4_0"](w)
        del w
        y = d_gemv("q4_0", x, wq, N, K)
        assert np.isfinite(y).all()
        tot_ref, tot_mag = 0.0, 0.0
        for lo in range(0, N, 16384):
            hi = min(N, lo + 16384)
            ref, mag = o.gemv_exact("q4_0", x, wq[lo:hi], hi - lo, K)
            assert (np.abs(y[lo:hi] - ref) <= o.gemv_bound(K, mag)).all()
            tot_ref += ref.sum()
            tot_mag += mag.sum()
        assert abs(float(np.sum(y.astype(np.float64))) - tot_ref) <= 2 * (K // 32 + 4) * 2.0 ** -24 * tot_mag


class TestModuleHostPath:
    """The pybind11 module (host arrays) on the same cases: it must equal the device entry point."""

    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    def test_module_equals_device_entry(self, fmt):
        import simd_ml_kernels as sk
        N, K = 300, 2048
        rng = np.random.default_rng(11)
        w = rng.standard_normal((N, K)).astype(np.float32)
        x = rng.standard_normal(K).astype(np.float32)
        wq = getattr(sk, f"quantize_{fmt}")(w)
        np.testing.assert_array_equal(wq, QUANT[fmt](w))
        y = getattr(sk, f"gemv_{fmt}")(x, wq, N, K)
        np.testing.assert_array_equal(y.view(np.uint32), d_gemv(fmt, x, wq, N, K).view(np.uint32))
        # unaligned host buffers, read-only (pinned) weights
        buf = np.empty(wq.size + 1, np.uint8)
        buf[1:] = wq.ravel()
        xbuf = np.empty(K + 1, np.float32)
        xbuf[1:] = x
        np.testing.assert_array_equal(getattr(sk, f"gemv_{fmt}")(xbuf[1:], buf[1:], N, K), y)
        ro = wq.copy()
        ro.setflags(write=False)
        for _ in range(2):
            np.testing.assert_array_equal(getattr(sk, f"gemv_{fmt}")(x, ro, N, K), y)

    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    def test_module_edge_cases(self, fmt):
        import simd_ml_kernels as sk
        gemv, q = getattr(sk, f"gemv_{fmt}"), getattr(sk, f"quantize_{fmt}")
        assert (gemv(np.ones(0, np.float32), np.zeros(0, np.uint8), 5, 0) == 0).all()
        assert gemv(np.ones(32, np.float32), np.zeros(0, np.uint8), 0, 32).shape == (0,)
        x = np.ones(64, np.float32)
        x[3] = np.nan
        assert np.isnan(gemv(x, q(np.ones((4, 64), np.float32)), 4, 64)).all()
        w = np.ones((2, 64), np.float32)
        w[0, 0] = np.inf
        with pytest.raises(sk.ArgumentError):
            q(w)

    def test_module_gemm_rows(self):
        import simd_ml_kernels as sk
        rng = np.random.default_rng(2)
        X = rng.standard_normal((32, 4096)).astype(np.float32)
        wq = sk.quantize_q4_0(rng.standard_normal((200, 4096)).astype(np.float32))
        Y = sk.gemm_q4_0(X, wq, 200, 4096)
        for m in (0, 7, 8, 31):
            np.testing.assert_array_equal(Y[m], sk.gemv_q4_0(X[m], wq, 200, 4096))
