"""CPU oracle for the decode-GEMV path.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, and only as the checker.  The product (libsmk_hip.so and the
simd_ml_kernels._core module) never imports, links or calls it.

Three layers:
  * ``lib()``: ctypes over liboracle.so, the plain-C restatement (smk_oracle.c).
  * numpy restatements that are independent of the C code (quantizers written
    with numpy's own float32 arithmetic, float64 exact sums and the reference's
    documented error bounds, the RMSNorm / RoPE / SiLU formulas of
    examples/llama/llama.py).
  * ``ref()``: ctypes over oracle/_ref/libsmk_ref.so, the REFERENCE's own kernel
    units compiled from /root/reference/src by oracle/Makefile (None when that
    library was never built).

Each function cites the reference file:line it restates.
"""

from __future__ import annotations

import ctypes
import math
import os
from functools import lru_cache

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
U32 = 2.0 ** -24  # unit roundoff of binary32

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i8p = ctypes.POINTER(ctypes.c_int8)
_i32p = ctypes.POINTER(ctypes.c_int32)


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


@lru_cache(maxsize=None)
def lib() -> ctypes.CDLL:
    path = os.path.join(HERE, "liboracle.so")
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
    L = ctypes.CDLL(path)
    L.smko_fp32_to_fp16.restype = ctypes.c_uint16
    L.smko_fp32_to_fp16.argtypes = [ctypes.c_float]
    L.smko_fp16_to_fp32.restype = ctypes.c_float
    L.smko_fp16_to_fp32.argtypes = [ctypes.c_uint16]
    for name in ("smko_quantize_q8_0_rows", "smko_quantize_q4_0_rows"):
        getattr(L, name).restype = ctypes.c_int
        getattr(L, name).argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _u8p]
    L.smko_quantize_x_q8.restype = ctypes.c_int
    L.smko_quantize_x_q8.argtypes = [_f32p, ctypes.c_int, _i8p, _f32p]
    for name in ("smko_gemv_q8_0", "smko_gemv_q4_0"):
        getattr(L, name).restype = None
        getattr(L, name).argtypes = [ctypes.c_int, ctypes.c_int, _f32p, _u8p, _f32p]
    for name in ("smko_block_sums_q8_0", "smko_block_sums_q4_0"):
        getattr(L, name).restype = None
        getattr(L, name).argtypes = [ctypes.c_int, ctypes.c_int, _i8p, _u8p, _i32p]
    L.smko_gemm_tb.restype = None
    L.smko_gemm_tb.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                               ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_float,
                               _f32p, ctypes.c_int]
    L.smko_silu.restype = None
    L.smko_silu.argtypes = [_f32p, _f32p, ctypes.c_int]
    L.smko_gemv_q4_0_simd.restype = None
    L.smko_gemv_q4_0_simd.argtypes = [ctypes.c_int, ctypes.c_int, _f32p, _u8p, _f32p]
    for name in ("smko_sgemm_tb_simd", "smko_sgemm_nn_simd"):
        getattr(L, name).restype = None
        getattr(L, name).argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, _f32p, ctypes.c_int,
                                     _f32p, ctypes.c_int, ctypes.c_float, _f32p, ctypes.c_int]
    L.smko_fast_exp.restype = ctypes.c_float
    L.smko_fast_exp.argtypes = [ctypes.c_float]
    for name in ("smko_silu_simd", "smko_softmax_simd"):
        getattr(L, name).restype = None
        getattr(L, name).argtypes = [_f32p, _f32p, ctypes.c_int]
    return L


@lru_cache(maxsize=None)
def ref() -> ctypes.CDLL | None:
    """The reference's own kernels (oracle/_ref/libsmk_ref.so) or None."""
    path = os.path.join(HERE, "_ref", "libsmk_ref.so")
    if not os.path.exists(path):
        return None
    R = ctypes.CDLL(path)
    R.ref_table_available.restype = ctypes.c_int
    R.ref_table_available.argtypes = [ctypes.c_int]
    R.ref_table_flags.restype = ctypes.c_char_p
    R.ref_table_flags.argtypes = [ctypes.c_int]
    R.ref_q8_0_path.restype = ctypes.c_char_p
    R.ref_q8_0_path.argtypes = [ctypes.c_int]
    for name in ("ref_gemv_q4_0", "ref_gemv_q8_0"):
        getattr(R, name).restype = ctypes.c_int
        getattr(R, name).argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _u8p, _f32p]
    R.ref_sgemm.restype = ctypes.c_int
    R.ref_sgemm.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                            ctypes.c_float, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                            ctypes.c_float, _f32p, ctypes.c_int]
    for name in ("ref_sgemm_f16", "ref_sgemm_bf16"):
        getattr(R, name).restype = ctypes.c_int
        getattr(R, name).argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_float, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                     ctypes.c_float, _f32p, ctypes.c_int]
    for name in ("ref_silu", "ref_softmax_row"):
        getattr(R, name).restype = ctypes.c_int
        getattr(R, name).argtypes = [ctypes.c_int, _f32p, _f32p, ctypes.c_int]
    for name in ("ref_quantize_q4_0", "ref_quantize_q8_0"):
        getattr(R, name).restype = ctypes.c_int
        getattr(R, name).argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _u8p]
    R.ref_quantize_x_q8.restype = ctypes.c_int
    R.ref_quantize_x_q8.argtypes = [_f32p, ctypes.c_int, _i8p, _f32p]
    R.ref_fp32_to_fp16.restype = ctypes.c_uint16
    R.ref_fp32_to_fp16.argtypes = [ctypes.c_float]
    R.ref_fp16_to_fp32.restype = ctypes.c_float
    R.ref_fp16_to_fp32.argtypes = [ctypes.c_uint16]
    R.ref_set_num_threads.restype = None
    R.ref_set_num_threads.argtypes = [ctypes.c_int]
    R.ref_get_num_threads.restype = ctypes.c_int
    R.ref_get_num_threads.argtypes = []
    return R


ISA = {"scalar": 0, "avx2": 1, "avx512": 2}


def ref_best_isa() -> str | None:
    """Widest reference table this CPU runs (the one kernels() would pick, dispatch.cpp:217-230)."""
    R = ref()
    if R is None:
        return None
    for name in ("avx512", "avx2", "scalar"):
        if R.ref_table_available(ISA[name]):
            return name
    return None


# ─── C restatement wrappers ─────────────────────────────────────────────────

def _rows_k(W: np.ndarray) -> tuple[np.ndarray, int, int]:
    W = np.ascontiguousarray(W, dtype=np.float32)
    K = W.shape[-1]
    rows = W.size // K if K else 0
    return W, rows, K


def quantize_q4_0(W: np.ndarray) -> np.ndarray:
    """quantize_q4_0_rows (q4_0_scalar.cpp:64-78) -> uint8 [..., K/32*18]; ValueError on rejection."""
    W, rows, K = _rows_k(W)
    out = np.zeros(W.shape[:-1] + (K // 32 * 18,), np.uint8)
    if not lib().smko_quantize_q4_0_rows(_p(W, _f32p), rows, K, _p(out, _u8p)):
        raise ValueError("quantize_q4_0: non-finite value or float16 scale overflow")
    return out


def quantize_q8_0(W: np.ndarray) -> np.ndarray:
    """quantize_q8_0_rows (q8_0_scalar.cpp:96-111) -> uint8 [..., K/32*34]; ValueError on rejection."""
    W, rows, K = _rows_k(W)
    out = np.zeros(W.shape[:-1] + (K // 32 * 34,), np.uint8)
    if not lib().smko_quantize_q8_0_rows(_p(W, _f32p), rows, K, _p(out, _u8p)):
        raise ValueError("quantize_q8_0: non-finite value or float16 scale overflow")
    return out


def quantize_x_q8(x: np.ndarray) -> tuple[np.ndarray, np.ndarray] | None:
    """quantize_x_q8 (q8_0_scalar.cpp:113-118): int8 quants [K] and FP32 scales [K/32]; None if x is not finite."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = x.shape[0]
    qs = np.zeros(K, np.int8)
    dx = np.zeros(K // 32, np.float32)
    if not lib().smko_quantize_x_q8(_p(x, _f32p), K, _p(qs, _i8p), _p(dx, _f32p)):
        return None
    return qs, dx


def gemv_q4_0(x: np.ndarray, Wq: np.ndarray, N: int, K: int) -> np.ndarray:
    """Scalar-table gemv_q4_0 semantics (q4_0_scalar.cpp:82-105 under q8_0_scalar.cpp:120-166)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    Wq = np.ascontiguousarray(Wq, dtype=np.uint8)
    y = np.zeros(N, np.float32)
    lib().smko_gemv_q4_0(N, K, _p(x, _f32p), _p(Wq, _u8p), _p(y, _f32p))
    return y


def gemv_q8_0(x: np.ndarray, Wq: np.ndarray, N: int, K: int) -> np.ndarray:
    """Scalar-table gemv_q8_0 semantics (q8_0_scalar.cpp:170-192)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    Wq = np.ascontiguousarray(Wq, dtype=np.uint8)
    y = np.zeros(N, np.float32)
    lib().smko_gemv_q8_0(N, K, _p(x, _f32p), _p(Wq, _u8p), _p(y, _f32p))
    return y


def block_sums(fmt: str, qs: np.ndarray, Wq: np.ndarray, N: int, K: int) -> np.ndarray:
    """Exact per-block int32 dot products [N, K/32] of x's Q8 quants against W's blocks."""
    qs = np.ascontiguousarray(qs, dtype=np.int8)
    Wq = np.ascontiguousarray(Wq, dtype=np.uint8)
    out = np.zeros((N, K // 32), np.int32)
    fn = lib().smko_block_sums_q4_0 if fmt == "q4_0" else lib().smko_block_sums_q8_0
    fn(N, K, _p(qs, _i8p), _p(Wq, _u8p), _p(out, _i32p))
    return out


ELEM = {"fp32": 0, "f16": 1, "bf16": 2}


def gemm_tb(fmt: str, A: np.ndarray, W: np.ndarray, alpha: float = 1.0, beta: float = 0.0,
            C: np.ndarray | None = None) -> np.ndarray:
    """Scalar table trans_b product (scalar_kernels.cpp:66-84): C = beta*C + alpha*A*W^T, sequential FP32 dots."""
    A = np.ascontiguousarray(A)
    W = np.ascontiguousarray(W)
    M, K = A.shape
    N = W.shape[0]
    out = np.zeros((M, N), np.float32) if C is None else np.array(C, np.float32, copy=True)
    lib().smko_gemm_tb(ELEM[fmt], M, N, K, alpha, A.ctypes.data, K, W.ctypes.data, K, beta, _p(out, _f32p), N)
    return out


def silu_scalar(x: np.ndarray) -> np.ndarray:
    """silu_scalar (scalar_kernels.cpp:196-198)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().smko_silu(_p(x, _f32p), _p(y, _f32p), x.size)
    return y


def gemv_q4_0_simd(x: np.ndarray, Wq: np.ndarray, N: int, K: int) -> np.ndarray:
    """The reference's SIMD-table Q4_0 GEMV order (q4_0_rows.hpp): bit-exact y."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(N, np.float32)
    lib().smko_gemv_q4_0_simd(N, K, _p(x, _f32p), _p(np.ascontiguousarray(Wq), _u8p), _p(y, _f32p))
    return y


def sgemm_tb_simd(A: np.ndarray, B: np.ndarray, alpha: float = 1.0) -> np.ndarray:
    """alpha * A @ B.T in the AVX-512 table's few-row order (avx512_gemm_packed.cpp:216-240)."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    M, K = A.shape
    N = B.shape[0]
    C = np.zeros((M, N), np.float32)
    lib().smko_sgemm_tb_simd(M, N, K, alpha, _p(A, _f32p), K, _p(B, _f32p), K, 0.0, _p(C, _f32p), N)
    return C


def sgemm_nn_simd(A: np.ndarray, B: np.ndarray, alpha: float = 1.0) -> np.ndarray:
    """alpha * A @ B in the AVX2 direct path's order (avx2_gemm_packed.cpp:151-201)."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    M, K = A.shape
    N = B.shape[1]
    C = np.zeros((M, N), np.float32)
    lib().smko_sgemm_nn_simd(M, N, K, alpha, _p(A, _f32p), K, _p(B, _f32p), N, 0.0, _p(C, _f32p), N)
    return C


def silu_simd(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().smko_silu_simd(_p(x, _f32p), _p(y, _f32p), x.size)
    return y


def softmax_simd(x: np.ndarray) -> np.ndarray:
    """Rows of x through softmax_row_avx2's order (softmax_avx2.cpp:95-186)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    n = x.shape[-1]
    for r in range(x.size // max(n, 1)):
        lib().smko_softmax_simd(_p(x.reshape(-1, n)[r], _f32p), _p(y.reshape(-1, n)[r], _f32p), n)
    return y


# ─── Independent numpy restatements ────────────────────────────────────────

def fp16_bits(x: np.ndarray) -> np.ndarray:
    """numpy's float16 cast (IEEE round to nearest even) as bit patterns."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def q8_0_quantize_numpy(w: np.ndarray) -> np.ndarray:
    """ggml quantize_row_q8_0_ref in numpy float32 (q8_0.hpp:7-16): d = amax/127,
    q = round(w*(1/d)) half away from zero (trunc and compare: np.round is half-even),
    q = 0 where 1/d overflows, scale float16 little-endian."""
    k = w.shape[-1]
    b = np.asarray(w, np.float32).reshape(-1, k // 32, 32)
    amax = np.abs(b).max(axis=2)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore", over="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    idv[np.isinf(idv)] = 0
    v = (b * idv[:, :, None]).astype(np.float32)
    t = np.trunc(v)
    r = v - t  # exact in float32 for |v| <= 127.5
    q = (t + (r >= 0.5) - (r <= -0.5)).astype(np.int8)
    out = np.empty(b.shape[:2] + (34,), np.uint8)
    out[:, :, :2] = d.astype("<f2").view(np.uint8).reshape(b.shape[:2] + (2,))
    out[:, :, 2:] = q.view(np.uint8)
    return out.reshape(w.shape[:-1] + (k // 32 * 34,))


def q4_0_quantize_numpy(w: np.ndarray) -> np.ndarray:
    """ggml quantize_row_q4_0_ref in numpy float32 (q4_0.hpp:7-21): the first value of
    largest magnitude sets d = max/-8; q = min(15, trunc(w*(1/d) + 8.5)), product and
    sum rounded separately; id = 0 where d = 0 or 1/d overflows."""
    k = w.shape[-1]
    b = np.asarray(w, np.float32).reshape(-1, k // 32, 32)
    a = np.abs(b)
    first = np.take_along_axis(b, a.argmax(axis=2)[:, :, None], axis=2)[:, :, 0]
    mx = np.where(a.max(axis=2) > 0, first, np.float32(0)).astype(np.float32)
    d = (mx / np.float32(-8)).astype(np.float32)
    with np.errstate(divide="ignore", over="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    idv[np.isinf(idv)] = 0
    v = (b * idv[:, :, None]).astype(np.float32)
    t = (v + np.float32(8.5)).astype(np.float32)
    q = np.minimum(np.trunc(t), 15).astype(np.uint8)
    out = np.empty(b.shape[:2] + (18,), np.uint8)
    out[:, :, :2] = d.astype("<f2").view(np.uint8).reshape(b.shape[:2] + (2,))
    out[:, :, 2:] = q[:, :, :16] | (q[:, :, 16:] << 4)
    return out.reshape(w.shape[:-1] + (k // 32 * 18,))


def q8_0_split(Wq: np.ndarray, n: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    """float16 scales (as float64 [n, k/32]) and int8 quants [n, k/32, 32] of Q8_0 bytes."""
    b = np.ascontiguousarray(Wq).reshape(n, k // 32, 34)
    d = np.ascontiguousarray(b[:, :, :2]).view("<f2")[:, :, 0].astype(np.float64)
    return d, np.ascontiguousarray(b[:, :, 2:]).view(np.int8)


def q4_0_split(Wq: np.ndarray, n: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    """float16 scales (float64 [n, k/32]) and signed quants q-8 (int8 [n, k/32, 32]) of Q4_0 bytes;
    byte j holds value j (low nibble) and value 16+j (high nibble), q4_0.hpp:7-11."""
    b = np.ascontiguousarray(Wq).reshape(n, k // 32, 18)
    d = np.ascontiguousarray(b[:, :, :2]).view("<f2")[:, :, 0].astype(np.float64)
    qs = b[:, :, 2:]
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=2).astype(np.int8) - np.int8(8)
    return d, q


def x_scales(x: np.ndarray) -> np.ndarray:
    """FP32 dx = max|x|/127 per block (q8_0.hpp:20-22)."""
    amax = np.abs(np.asarray(x, np.float32)).reshape(-1, 32).max(axis=1)
    return (amax / np.float32(127)).astype(np.float32)


def gemv_exact(fmt: str, x: np.ndarray, Wq: np.ndarray, N: int, K: int) -> tuple[np.ndarray, np.ndarray]:
    """The GEMV of the quantized operands taken exactly (float64, int64 block sums) and the
    bound's magnitude sum_b |dw*dx| * sum_i |qw*qx| (restates _cli.py:157-189)."""
    dw, qw = (q4_0_split if fmt == "q4_0" else q8_0_split)(Wq, N, K)
    _, qx = q8_0_split(q8_0_quantize_numpy(np.asarray(x, np.float32)), 1, K)
    sc = dw * x_scales(x).astype(np.float64)[None, :]
    prod = qw.astype(np.int64) * qx.astype(np.int64)
    return ((prod.sum(axis=2).astype(np.float64) * sc).sum(axis=1),
            (np.abs(prod).sum(axis=2).astype(np.float64) * np.abs(sc)).sum(axis=1))


def gemv_bound(K: int, mag: np.ndarray) -> np.ndarray:
    """|y - y64| <= 2*(K/32 + 4)*u*mag (q4_0.hpp:30, q8_0.hpp:26)."""
    return 2 * (K // 32 + 4) * U32 * mag + 1e-300


def gemm_bound(K: int, absprod: np.ndarray) -> np.ndarray:
    """|C - C64| <= 2(K+2)u * (|A||W|^T) (test_precision.py:212-220)."""
    return 2 * (K + 2) * U32 * absprod


def to_bf16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (test_precision.py:176-178's rule)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def silu64(x: np.ndarray) -> np.ndarray:
    """SiLU in float64 (the selftest's reference, _cli.py:313-314)."""
    x = np.asarray(x, np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        return x / (1.0 + np.exp(-x))


def softmax64(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


# ─── Llama decode formulas (examples/llama/llama.py) ───────────────────────

def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """llama.py:184-187: var = mean(x*x) in float32 (numpy pairwise sum), scale 1/sqrt computed
    in float64 then rounded to float32, w * (x * scale)."""
    var = np.mean(x * x, dtype=np.float32)
    return weight * (x * np.float32(1.0 / math.sqrt(float(var) + eps)))


def numpy_sum_f32(a: np.ndarray, bufsize: int = 8192) -> np.float32:
    """np.add.reduce of a contiguous float32 vector, restated: the reduction runs over chunks
    of the ufunc buffer size (8192), each chunk summed pairwise and the chunk sums added in
    order to -0.0.  The model the GPU RMSNorm follows; checked against np.add.reduce."""
    a = np.ascontiguousarray(a, np.float32)
    r = np.float32(-0.0)
    for s in range(0, a.size, bufsize):
        r = np.float32(r + pairwise_sum_f32(a[s:s + bufsize]))
    return r


def pairwise_sum_f32(a: np.ndarray) -> np.float32:
    """numpy's float32 pairwise summation (numpy/_core/src/umath/loops_utils.h.src,
    pairwise_sum): n < 8 sequential from 0; n <= 128 eight interleaved accumulators combined
    ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) then the n % 8 tail in order; larger n split at
    n2 = n/2 - (n/2) % 8."""
    a = np.ascontiguousarray(a, np.float32)

    def rec(lo: int, n: int) -> np.float32:
        if n < 8:
            r = np.float32(0)
            for i in range(n):
                r = np.float32(r + a[lo + i])
            return r
        if n <= 128:
            r = [a[lo + k] for k in range(8)]
            i = 8
            while i < n - (n % 8):
                for k in range(8):
                    r[k] = np.float32(r[k] + a[lo + i + k])
                i += 8
            res = np.float32(np.float32(np.float32(r[0] + r[1]) + np.float32(r[2] + r[3])) +
                             np.float32(np.float32(r[4] + r[5]) + np.float32(r[6] + r[7])))
            while i < n:
                res = np.float32(res + a[lo + i])
                i += 1
            return res
        n2 = n // 2
        n2 -= n2 % 8
        return np.float32(rec(lo, n2) + rec(lo + n2, n - n2))

    return rec(0, a.size)


def rms_norm64(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    x64 = np.asarray(x, np.float64)
    return np.asarray(weight, np.float64) * x64 / math.sqrt(float(np.mean(x64 * x64)) + eps)


def rope_inv_freq(head_dim: int, theta: float, rope_scaling: dict | None) -> np.ndarray:
    """llama.py:131-159 (transformers' default / llama3 inverse frequencies in float32)."""
    exponent = np.arange(0, head_dim, 2, dtype=np.int64).astype(np.float32) / np.float32(head_dim)
    inv_freq = (np.float32(1.0) / (np.float32(theta) ** exponent)).astype(np.float32)
    kind = None if rope_scaling is None else rope_scaling.get("rope_type", rope_scaling.get("type"))
    if kind in (None, "default"):
        return inv_freq
    if kind != "llama3":
        raise ValueError(f"rope_scaling {kind!r} not implemented")
    factor = rope_scaling["factor"]
    low, high = rope_scaling["low_freq_factor"], rope_scaling["high_freq_factor"]
    old_len = rope_scaling["original_max_position_embeddings"]
    low_wl, high_wl = old_len / low, old_len / high
    wavelen = (np.float32(2 * math.pi) / inv_freq).astype(np.float32)
    scaled = np.where(wavelen > low_wl, inv_freq / np.float32(factor), inv_freq).astype(np.float32)
    smooth = ((np.float32(old_len) / wavelen - np.float32(low)) / np.float32(high - low)).astype(np.float32)
    smoothed = ((1 - smooth) * scaled / np.float32(factor) + smooth * scaled).astype(np.float32)
    medium = ~(wavelen < high_wl) & ~(wavelen > low_wl)
    return np.where(medium, smoothed, scaled).astype(np.float32)


def rope_cos_sin(inv_freq: np.ndarray, pos: int) -> tuple[np.ndarray, np.ndarray]:
    """llama.py:162-166: cos/sin [head_dim] with the halves repeated."""
    angles = (np.float32(pos) * inv_freq).astype(np.float32)
    emb = np.concatenate([angles, angles])
    return np.cos(emb), np.sin(emb)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, interleaved: bool) -> np.ndarray:
    """llama.py:387-396 (interleaved pairs 2i, 2i+1) and :169-178 (HF rotate_half)."""
    if interleaved:
        half = x.shape[-1] // 2
        a, b = x[:, 0::2], x[:, 1::2]
        c, s = cos[:half], sin[:half]
        out = np.empty_like(x)
        out[:, 0::2] = a * c - b * s
        out[:, 1::2] = b * c + a * s
        return out
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[:, half:], x[:, :half]], axis=-1)
    return x * cos + rot * sin


def synthetic(seed: int, shapes: list[tuple[int, ...]], scales: list[float]) -> list[np.ndarray]:
    """Seeded inputs: rng = default_rng(seed); each array standard normal float32 times its scale,
    drawn in order (x first, then W), as the benchmark recipe of the measurement plan."""
    rng = np.random.default_rng(seed)
    out = []
    for shape, s in zip(shapes, scales):
        a = rng.standard_normal(shape, dtype=np.float32)
        if s != 1.0:
            a *= np.float32(s)
        out.append(a)
    return out
