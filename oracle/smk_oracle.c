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
 * |f| >= 65520 -> infinity.  Semantics of q8_0_scalar.cpp:65-81. */
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

/* binary16 -> binary32, exact (q8_0_scalar.cpp:83-94). */
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

/* One Q8_0 block (ggml quantize_row_q8_0_ref; q8_0_scalar.cpp:36-61):
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

/* One Q4_0 block (ggml quantize_row_q4_0_ref; q4_0_scalar.cpp:23-60): max = the first
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

/* The driver's rules (q8_0_scalar.cpp:120-166): N <= 0 writes nothing, K <= 0 gives
 * zeros, a non-finite x gives NaN everywhere; blocks summed in order, one rounding per
 * step: acc += float(isum) * (dw * dx) (q8_0_scalar.cpp:170-186, q4_0_scalar.cpp:82-99). */
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

/* ─── The reference's SIMD-path arithmetic orders ───────────────────────────
 * The AVX2 / AVX-VNNI / AVX512-VNNI tables share one Q4_0 row loop (q4_0_rows.hpp:71-167,
 * eight rows per group in every unit: q4_0_avx2.cpp:31, q4_0_avxvnni.cpp:28,
 * q4_0_avx512vnni.cpp:30).  Rows are walked in pairs, one row per 128-bit half of a YMM
 * register: lane k (0..3) of a row holds the exact integer dot of values {4k..4k+3} (low
 * nibbles) and {16+4k..16+4k+3} (high nibbles) with x's quants, -8 times x's sum over the
 * same eight values as its start, and accumulates fma(float(dot), fp16(d)*dx, acc) over the
 * blocks in order; y = (acc0 + acc2) + (acc1 + acc3) (q4_hsum4).  The last row of an odd N
 * takes q4_row_single: eight lanes, lane k < 4 over values {4k..4k+3}, lane k >= 4 over
 * {16+4(k-4)..}; y = hsum4(acc[0..3] + acc[4..7]). */
static int32_t q4_lane_dot(const uint8_t* qbytes, const int8_t* xb, const int* vals, int nvals) {
    int32_t s = 0, sx = 0;
    for (int i = 0; i < nvals; ++i) {
        const int v = vals[i];
        const int q = v < 16 ? (qbytes[v] & 0x0f) : (qbytes[v - 16] >> 4);
        s += q * xb[v];
        sx += xb[v];
    }
    return s - 8 * sx;
}

void smko_gemv_q4_0_simd(int N, int K, const float* x, const uint8_t* Wq, float* y) {
    if (N <= 0) return;
    if (K <= 0) { for (int n = 0; n < N; ++n) y[n] = 0.0f; return; }
    const int nb = K / 32;
    int8_t qs[K];
    float dx[nb];
    if (!smko_quantize_x_q8(x, K, qs, dx)) {
        for (int n = 0; n < N; ++n) y[n] = NAN;
        return;
    }
    for (int n = 0; n < N; ++n) {
        const int single = (N & 1) && n == N - 1;
        const int lanes = single ? 8 : 4;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int b = 0; b < nb; ++b) {
            const uint8_t* blk = Wq + ((size_t)n * nb + b) * 18;
            const float s = scale_of(blk) * dx[b];
            for (int k = 0; k < lanes; ++k) {
                int vals[8], nv = 0;
                if (!single) {
                    for (int j = 0; j < 4; ++j) vals[nv++] = 4 * k + j;
                    for (int j = 0; j < 4; ++j) vals[nv++] = 16 + 4 * k + j;
                } else {
                    const int base = k < 4 ? 4 * k : 16 + 4 * (k - 4);
                    for (int j = 0; j < 4; ++j) vals[nv++] = base + j;
                }
                const int32_t d = q4_lane_dot(blk + 2, qs + 32 * b, vals, nv);
                acc[k] = fmaf((float)d, s, acc[k]);
            }
        }
        if (single)
            for (int k = 0; k < 4; ++k) acc[k] = acc[k] + acc[k + 4];
        y[n] = (acc[0] + acc[2]) + (acc[1] + acc[3]);
    }
}

/* AVX-512 table, trans_b with a few rows (avx512_gemm_packed.cpp:216-240): per output, two
 * 16-lane accumulators over steps of 32 (lane l of the first takes p + l, of the second
 * p + 16 + l; a masked tail step for K % 32), fused multiply-adds; then the 16 sums of the two
 * accumulators are reduced by halves (lanes i and i + 8, then i and i + 4, then i and i + 2,
 * then the last two: _mm512_reduce_add_ps); c = c*beta-scaled + alpha * sum. */
static float reduce16(const float* v) {
    float t8[8], t4[4], t2[2];
    for (int i = 0; i < 8; ++i) t8[i] = v[8 + i] + v[i];
    for (int i = 0; i < 4; ++i) t4[i] = t8[4 + i] + t8[i];
    t2[0] = t4[0] + t4[2];
    t2[1] = t4[1] + t4[3];
    return t2[0] + t2[1];
}

void smko_sgemm_tb_simd(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                        float beta, float* C, int ldc) {
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
            const float* a = A + (size_t)i * lda;
            const float* b = B + (size_t)j * ldb;
            float acc0[16], acc1[16], v[16];
            for (int l = 0; l < 16; ++l) acc0[l] = acc1[l] = 0.0f;
            for (int p = 0; p < K; p += 32)
                for (int l = 0; l < 16; ++l) {
                    if (p + l < K) acc0[l] = fmaf(a[p + l], b[p + l], acc0[l]);
                    if (p + 16 + l < K) acc1[l] = fmaf(a[p + 16 + l], b[p + 16 + l], acc1[l]);
                }
            for (int l = 0; l < 16; ++l) v[l] = acc0[l] + acc1[l];
            float* c = C + (size_t)i * ldc + j;
            *c = fmaf(alpha, reduce16(v), *c);
        }
}

/* AVX2 direct path without transposes (avx2_gemm_packed.cpp:151-201, 599-620): per output one
 * fused multiply-add chain over p in order, then c = fma(acc, alpha, c-prescaled-by-beta). */
void smko_sgemm_nn_simd(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                        float beta, float* C, int ldc) {
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
            for (int p = 0; p < K; ++p) acc = fmaf(A[(size_t)i * lda + p], B[(size_t)p * ldb + j], acc);
            float* c = C + (size_t)i * ldc + j;
            *c = fmaf(acc, alpha, *c);
        }
}

/* fast_exp_avx2 (simd_math.hpp:63-117): clamp to +-88.3762626647949, k = floor(z*log2e + 0.5)
 * (one fused multiply-add), f = z - k*ln2_hi - k*ln2_lo (two fused steps), a degree-6 Horner
 * polynomial in fused multiply-adds, times 2^k built from the exponent bits.  min/max keep
 * the second operand when the first is NaN, as vminps / vmaxps. */
float smko_fast_exp(float z) {
    const float hi = 88.3762626647949f, lo = -88.3762626647949f;
    z = z < hi ? z : hi;
    z = z > lo ? z : lo;
    const float kf = floorf(fmaf(z, 1.44269504088896341f, 0.5f));
    const int ki = (int)kf;
    float f = fmaf(-kf, 0.693359375f, z);
    f = fmaf(-kf, -2.12194440e-4f, f);
    float p = 1.3890048347e-3f;
    p = fmaf(p, f, 8.3338161260e-3f);
    p = fmaf(p, f, 4.1666668259e-2f);
    p = fmaf(p, f, 1.6666667163e-1f);
    p = fmaf(p, f, 0.5f);
    p = fmaf(p, f, 1.0f);
    p = fmaf(p, f, 1.0f);
    return p * u2f((uint32_t)(ki + 127) << 23);
}

/* silu_avx2 (silu_avx2.cpp:38-45): x / (1 + fast_exp(-x)), the denominator +inf when -x > 88. */
void smko_silu_simd(const float* in, float* out, int n) {
    for (int i = 0; i < n; ++i) {
        const float x = in[i], nx = -x;
        float d = 1.0f + smko_fast_exp(nx);
        if (nx > 88.0f) d = INFINITY;
        out[i] = x / d;
    }
}

/* softmax_row_avx2 (softmax_avx2.cpp:95-186): NaN rows as the scalar kernel; then per full
 * group of 8 e = fast_exp(x - max) stored as float, its double added to eight running double
 * sums (lane j of the group into sum j); those eight are added in order (s0+s1+...+s7) to 0;
 * the last n % 8 values use e = exp(double(x - max)) (glibc) added in order; every output is
 * then multiplied by float(1 / sum). */
void smko_softmax_simd(const float* in, float* out, int n) {
    if (n <= 0) return;
    float mx = in[0];
    int bad = 0;
    for (int i = 0; i < n; ++i) {
        const uint32_t u = f2u(in[i]);
        bad |= (u & 0x7fffffffu) > 0x7f800000u || u == 0x7f800000u;
        if (in[i] > mx) mx = in[i];
    }
    if (bad || f2u(mx) == 0xff800000u) {
        for (int i = 0; i < n; ++i) out[i] = NAN;
        return;
    }
    double lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; ++j) {
            const float e = smko_fast_exp(in[i + j] - mx);
            out[i + j] = e;
            lanes[j] += (double)e;
        }
    double sum = 0.0;
    sum += lanes[0] + lanes[1] + lanes[2] + lanes[3] + lanes[4] + lanes[5] + lanes[6] + lanes[7];
    for (; i < n; ++i) {
        const double e = exp((double)(in[i] - mx));
        out[i] = (float)e;
        sum += e;
    }
    const float inv = (float)(1.0 / sum);
    for (int j = 0; j < n; ++j) out[j] *= inv;
}
