/*
 * smk_oracle.c -- CPU oracle for the decode-GEMV path.  TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's scalar semantics.  It is the checker
 * for the HIP product, never the product: only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load it.  Built with -O2 -ffp-contract=off and
 * no fast-math (oracle/Makefile), so every float operation below is one IEEE
 * binary32 operation, as in the reference's scalar unit
 * (/root/reference/CMakeLists.txt:183-190).
 *
 * What pins each function (tests/test_oracle.py):
 *   fp32<->fp16        every binary16 value, every midpoint +-1 ulp, overflow, NaN
 *                      (recipe of tests/test_q8_0.cpp:40-67), numpy's float16 cast,
 *                      and the reference's own fp32_to_fp16 built in oracle/_ref.
 *   quantize_q4_0      the committed llama.cpp v0.7.0 fixture (tests/golden), the
 *                      special blocks of test_q4_0.cpp:84-130 / test_precision.py:721-730,
 *                      an independent numpy restatement, and oracle/_ref.
 *   quantize_q8_0/x    special rows of test_precision.py:499-528, numpy (np.round is
 *                      half-even, so the restatement uses trunc-and-compare), oracle/_ref.
 *   block sums         brute force in int64 numpy.
 *   gemv_q{4,8}_0      the float64 exact sum with the bound of q4_0.hpp:30 / q8_0.hpp:26,
 *                      and bit-for-bit equality with the reference's scalar table (oracle/_ref).
 *   gemm_tb            float64 product with the bound 2(K+2)u|A||W| (test_precision.py:212-220)
 *                      and bit equality with the reference scalar table (oracle/_ref).
 *   silu               float64 formula with 1e-35 + 1e-6|ref| and the special values.
 */
#include "smk_oracle.h"

#include <math.h>
#include <string.h>

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* binary32 -> binary16, round to nearest even; NaN -> 0x7e00 with the sign,
 * |f| >= 65520 -> infinity.  Semantics of q8_0_scalar.cpp:260-276. */
uint16_t smko_fp32_to_fp16(float f) {
    const uint32_t u = f2u(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;          /* NaN */
    if (a >= 0x477ff000u) return sign | 0x7c00u;         /* >= 65520 (and inf) */
    if (a < 0x33000000u) return sign;                    /* < 2^-25: rounds to zero */
    const int e = (int)(a >> 23) - 127;                  /* a is normal here */
    const uint32_t m = (a & 0x7fffffu) | 0x800000u;      /* 24-bit significand */
    /* Normal results keep 11 bits (drop 13); subnormal results are multiples of 2^-24. */
    const int drop = e >= -14 ? 13 : 13 + (-14 - e);     /* 13 .. 24 */
    uint32_t q = m >> drop;
    const uint32_t rem = m & ((1u << drop) - 1u), half = 1u << (drop - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    /* q carries the implicit bit for normals: adding it bumps the exponent field by one. */
    const uint32_t h = (e >= -14 ? (uint32_t)(e + 14) << 10 : 0u) + q;
    return sign | (uint16_t)h;
}

/* binary16 -> binary32, exact (q8_0_scalar.cpp:278-289). */
float smko_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        const float mag = (float)m * 0x1p-24f;           /* exact: m < 2^10, power-of-two scale */
        return (h & 0x8000u) ? -mag : mag;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

static int finite_bits(float v) { return (f2u(v) & 0x7f800000u) != 0x7f800000u; }

static void store_scale(uint8_t* out, uint16_t h) {
    out[0] = (uint8_t)(h & 0xffu);
    out[1] = (uint8_t)(h >> 8);
}

/* One Q8_0 block (ggml quantize_row_q8_0_ref; q8_0_scalar.cpp:237-256):
 * d = amax/127, q = roundf(w * (1/d)) half away from zero, q = 0 when 1/d overflows. */
static int q8_block(const float* w, int8_t* q, float* d_out) {
    float amax = 0.0f;
    int finite = 1;
    for (int j = 0; j < 32; ++j) {
        finite &= finite_bits(w[j]);
        const float a = fabsf(w[j]);
        if (a > amax) amax = a;
    }
    if (!finite) return 0;
    const float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    if (isinf(id)) id = 0.0f;
    for (int j = 0; j < 32; ++j) q[j] = (int8_t)roundf(w[j] * id);
    *d_out = d;
    return 1;
}

int smko_quantize_q8_0_rows(const float* W, int N, int K, uint8_t* out) {
    const int nb = K / 32;
    for (int n = 0; n < N; ++n)
        for (int b = 0; b < nb; ++b, out += 34) {
            float d;
            if (!q8_block(W + (size_t)n * K + 32 * b, (int8_t*)(out + 2), &d)) return 0;
            const uint16_t h = smko_fp32_to_fp16(d);
            if ((h & 0x7fffu) == 0x7c00u) return 0;
            store_scale(out, h);
        }
    return 1;
}

int smko_quantize_x_q8(const float* x, int K, int8_t* qs, float* dx) {
    for (int b = 0; b < K / 32; ++b)
        if (!q8_block(x + 32 * b, qs + 32 * b, dx + b)) return 0;
    return 1;
}

/* One Q4_0 block (ggml quantize_row_q4_0_ref; q4_0_scalar.cpp:427-464): max = the first
 * value of largest magnitude, d = max / -8, q = min(15, trunc(w*id + 8.5)) with the
 * product and the sum rounded separately, id = 0 when d = 0 or 1/d overflows. */
static int q4_block(const float* w, uint8_t* qs, float* d_out) {
    float amax = 0.0f, max = 0.0f;
    int finite = 1;
    for (int j = 0; j < 32; ++j) {
        finite &= finite_bits(w[j]);
        const float a = fabsf(w[j]);
        if (a > amax) { amax = a; max = w[j]; }
    }
    if (!finite) return 0;
    const float d = max / -8.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    if (isinf(id)) id = 0.0f;
    uint8_t q[32];
    for (int j = 0; j < 32; ++j) {
        const float v = w[j] * id;
        const float t = v + 8.5f;
        const int iq = (int)t;          /* t in (0, 17): truncation toward zero */
        q[j] = (uint8_t)(iq < 15 ? iq : 15);
    }
    for (int j = 0; j < 16; ++j) qs[j] = (uint8_t)(q[j] | (q[16 + j] << 4));
    *d_out = d;
    return 1;
}

int smko_quantize_q4_0_rows(const float* W, int N, int K, uint8_t* out) {
    const int nb = K / 32;
    for (int n = 0; n < N; ++n)
        for (int b = 0; b < nb; ++b, out += 18) {
            float d;
            if (!q4_block(W + (size_t)n * K + 32 * b, out + 2, &d)) return 0;
            const uint16_t h = smko_fp32_to_fp16(d);
            if ((h & 0x7fffu) == 0x7c00u) return 0;
            store_scale(out, h);
        }
    return 1;
}

static float scale_of(const uint8_t* blk) { return smko_fp16_to_fp32((uint16_t)(blk[0] | (blk[1] << 8))); }

static int32_t q8_isum(const uint8_t* blk, const int8_t* p) {
    const int8_t* q = (const int8_t*)(blk + 2);
    int32_t s = 0;
    for (int i = 0; i < 32; ++i) s += (int32_t)q[i] * p[i];
    return s;
}

static int32_t q4_isum(const uint8_t* blk, const int8_t* p) {
    const uint8_t* q = blk + 2;
    int32_t s = 0;
    for (int j = 0; j < 16; ++j)
        s += ((int32_t)(q[j] & 0x0f) - 8) * p[j] + ((int32_t)(q[j] >> 4) - 8) * p[16 + j];
    return s;
}

void smko_block_sums_q8_0(int N, int K, const int8_t* qs, const uint8_t* Wq, int32_t* out) {
    const int nb = K / 32;
    for (int n = 0; n < N; ++n)
        for (int b = 0; b < nb; ++b)
            out[(size_t)n * nb + b] = q8_isum(Wq + ((size_t)n * nb + b) * 34, qs + 32 * b);
}

void smko_block_sums_q4_0(int N, int K, const int8_t* qs, const uint8_t* Wq, int32_t* out) {
    const int nb = K / 32;
    for (int n = 0; n < N; ++n)
        for (int b = 0; b < nb; ++b)
            out[(size_t)n * nb + b] = q4_isum(Wq + ((size_t)n * nb + b) * 18, qs + 32 * b);
}

/* The driver's rules (q8_0_scalar.cpp:315-361): N <= 0 writes nothing, K <= 0 gives
 * zeros, a non-finite x gives NaN everywhere; blocks summed in order, one rounding per
 * step: acc += float(isum) * (dw * dx) (q8_0_scalar.cpp:365-381, q4_0_scalar.cpp:486-503). */
static void gemv_blocks(int N, int K, const float* x, const uint8_t* Wq, float* y, int q4) {
    if (N <= 0) return;
    if (K <= 0) { for (int n = 0; n < N; ++n) y[n] = 0.0f; return; }
    const int nb = K / 32, bb = q4 ? 18 : 34;
    int8_t qs[K];
    float dx[nb];
    if (!smko_quantize_x_q8(x, K, qs, dx)) {
        for (int n = 0; n < N; ++n) y[n] = NAN;
        return;
    }
    for (int n = 0; n < N; ++n) {
        const uint8_t* blk = Wq + (size_t)n * nb * bb;
        float acc = 0.0f;
        for (int b = 0; b < nb; ++b, blk += bb) {
            const int32_t s = q4 ? q4_isum(blk, qs + 32 * b) : q8_isum(blk, qs + 32 * b);
            const float sc = scale_of(blk) * dx[b];
            acc += (float)s * sc;
        }
        y[n] = acc;
    }
}

void smko_gemv_q8_0(int N, int K, const float* x, const uint8_t* Wq, float* y) { gemv_blocks(N, K, x, Wq, y, 0); }
void smko_gemv_q4_0(int N, int K, const float* x, const uint8_t* Wq, float* y) { gemv_blocks(N, K, x, Wq, y, 1); }

static float load_elem(int elem, const void* base, size_t i) {
    if (elem == 0) return ((const float*)base)[i];
    const uint16_t h = ((const uint16_t*)base)[i];
    if (elem == 1) return smko_fp16_to_fp32(h);
    return u2f((uint32_t)h << 16);
}

/* Scalar table trans_b GEMM (scalar_kernels.cpp:66-84, 140-179): C = beta*C (beta = 0
 * writes zeros), then c[j] += alpha * acc with acc a sequential fp32 dot product. */
void smko_gemm_tb(int elem, int M, int N, int K, float alpha, const void* A, int lda, const void* B,
                  int ldb, float beta, float* C, int ldc) {
    if (M <= 0 || N <= 0 || K < 0) return;
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            float* c = C + (size_t)i * ldc + j;
            if (beta == 0.0f) *c = 0.0f;
            else if (beta != 1.0f) *c *= beta;
        }
    if (K == 0) return;
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            float acc = 0.0f;
            for (int p = 0; p < K; ++p)
                acc += load_elem(elem, A, (size_t)i * lda + p) * load_elem(elem, B, (size_t)j * ldb + p);
            C[(size_t)i * ldc + j] += alpha * acc;
        }
}

/* silu_scalar (scalar_kernels.cpp:196-198): x / (1 + exp(-x)) with libm. */
void smko_silu(const float* in, float* out, int n) {
    for (int i = 0; i < n; ++i) out[i] = in[i] / (1.0f + expf(-in[i]));
}
