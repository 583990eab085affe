// gemv_lowp.hip -- C = beta*C + alpha * A * B^T for FP32 / FP16 / BF16 B stored [N, K], for gfx950.
//
// The reference's trans_b dot path (avx2_gemm_packed.cpp:358-448, 680-732, and the scalar
// gemm_rows_tb, scalar_kernels.cpp:66-84): the M <= 8 rows of A are widened to FP32 once,
// every element of B is read once and widened in registers, FP32 fused multiply-adds.
//
// Stream kernel (rows 16-byte aligned, K a multiple of 8 elements): LPR lanes share a row of
// B and each loads 16 bytes per step (8 fp16/bf16 or 4+4 fp32 values).  FP32: A is staged in
// LDS as FP32 in K tiles, in two planes of float4 so that lanes read consecutive 16-byte
// entries, and every product is one FMA.  FP16 / BF16: A is staged as it is stored (8 values of
// 16 bits per 16-byte entry) and each pair of products is one v_dot2_f32_f16 / v_dot2_f32_bf16
// (exact products: 11- or 8-bit significands; FP32 sums), half the VALU of widening each value
// first -- which BF16 needs two instructions for (a shift or a mask), FP16 one (v_fma_mix).
// Everything else (odd K, unaligned rows, M > 8) takes a plain one-thread-per-output kernel.
#include "device_common.hpp"
#include "launch.hpp"

#include <algorithm>
#include <atomic>

namespace smk {
namespace {

constexpr int kThreads = 256;
// Diagnostics settings (set_lowp_tuning), read by every launch.
std::atomic<int> g_lowp_lpr{0}, g_lowp_unroll{0};

template <int E>
__device__ __forceinline__ float elem_to_float(const void* base, size_t i) {
    if constexpr (E == 0) return static_cast<const float*>(base)[i];
    else if constexpr (E == 1) return half_bits_to_float(static_cast<const uint16_t*>(base)[i]);
    else return bf16_bits_to_float(static_cast<const uint16_t*>(base)[i]);
}

// 16 bytes of a row of B as loaded (8 fp16 / bf16 values, or 4 fp32), widened at use.
template <int E>
__device__ __forceinline__ void widen(const u32x4& t, float* v) {
    const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (E == 0) {
            v[i] = __uint_as_float(w[i]);
        } else if constexpr (E == 1) {
            v[2 * i] = half_bits_to_float(w[i]);
            v[2 * i + 1] = half_bits_to_float(w[i] >> 16);
        } else {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
}

// acc + a.lo * b.lo + a.hi * b.hi for two packed FP16 (E = 1) or BF16 (E = 2) values each.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
template <int E>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    if constexpr (E == 1)
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc, false);
    else
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc, false);
}

// LPR lanes share a row; a lane takes 8-element groups j, j + LPR, ... of its U rows.  The
// loads of the next D groups are issued before the current D groups' FMAs (two register
// buffers), every load unconditional from a clamped row and group so the compiler's wait
// counts stay exact.  FP32 B takes two 16-byte loads per group.  B is read with non-temporal
// loads: the LPR lanes of a row read LPR * 16 contiguous bytes, whole lines that no later
// load touches (measured on MI355X, f16 4096x14336 23.0 -> 20.6 us, 14336x4096 22.6 -> 21.1).
template <int E, int LPR, int U, int MT, int D>
__global__ __launch_bounds__(kThreads) void gemv_lowp_kernel(int M, int N, int K, float alpha,
                                                             const void* __restrict__ A, int lda,
                                                             const void* __restrict__ B, int ldb, float beta,
                                                             float* __restrict__ C, int ldc, int kt, int a_vec) {
    constexpr int G = kWave / LPR;
    constexpr int kRowsPerWg = 4 * G * U;
    constexpr int L = E == 0 ? 2 : 1;             // 16-byte loads per 8-element group
    constexpr size_t kEs = E == 0 ? 4 : 2;
    extern __shared__ __align__(16) float4 xs[];  // FP32: [MT][2][kt/8] float4; else [MT][kt/8] uint4
    u32x4* const xh = reinterpret_cast<u32x4*>(xs);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int g = lane / LPR, j = lane % LPR;
    const int rb = blockIdx.x * kRowsPerWg + wave * G * U + g;
    const int groups_max = kt / 8;
    const char* rows[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
        rows[u] = static_cast<const char*>(B) + static_cast<size_t>(min(rb + u * G, N - 1)) * ldb * kEs;

    float acc[U][MT];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[u][m] = 0.0f;

    for (int k0 = 0; k0 < K; k0 += kt) {
        const int klen = min(kt, K - k0);
        const int groups = klen / 8;
        const int steps = (groups + LPR - 1) / LPR;  // groups of this lane: c = j + i * LPR, i < steps
        auto load = [&](int i0, u32x4 (&w)[D][U][L]) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const int c = min(j + (i0 + d) * LPR, groups - 1);
#pragma unroll
                for (int u = 0; u < U; ++u)
#pragma unroll
                    for (int h = 0; h < L; ++h)
                        w[d][u][h] = __builtin_nontemporal_load(
                            reinterpret_cast<const u32x4*>(rows[u] + (static_cast<size_t>(k0) + 8 * c) * kEs) + h);
            }
        };
        u32x4 wa[D][U][L], wb[D][U][L];
        load(0, wa);  // both buffers are issued before the A tile is staged (whose loads wait
        load(D, wb);  // for everything issued earlier)
        __syncthreads();
        // A tile: 8-element groups, four loaded per thread before any is stored (16-byte loads
        // when A's rows are 16-byte aligned), so its loads wait together once.
        const int ng = M * groups;
        if constexpr (E != 0) {
            for (int i0 = threadIdx.x; i0 < ng; i0 += 4 * kThreads) {
                u32x4 v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int i = min(i0 + q * kThreads, ng - 1);
                    const int m = i / groups, grp = i - m * groups;
                    const size_t base = static_cast<size_t>(m) * lda + k0 + 8 * grp;
                    if (a_vec) {
                        v[q] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(A) + base);
                    } else {
                        const uint16_t* p = static_cast<const uint16_t*>(A) + base;
                        v[q] = u32x4{p[0] | (static_cast<uint32_t>(p[1]) << 16), p[2] | (static_cast<uint32_t>(p[3]) << 16),
                                     p[4] | (static_cast<uint32_t>(p[5]) << 16), p[6] | (static_cast<uint32_t>(p[7]) << 16)};
                    }
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int i = i0 + q * kThreads;
                    if (i < ng) {
                        const int m = i / groups, grp = i - m * groups;
                        xh[m * groups_max + grp] = v[q];
                    }
                }
            }
        }
        for (int i0 = threadIdx.x; E == 0 && i0 < ng; i0 += 4 * kThreads) {
            float v[4][8];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = min(i0 + q * kThreads, ng - 1);
                const int m = i / groups, grp = i - m * groups;
                const size_t base = static_cast<size_t>(m) * lda + k0 + 8 * grp;
                if (a_vec) {
                    const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const char*>(A) + base * kEs);
                    widen<E>(p[0], v[q]);
                    if constexpr (L == 2) widen<E>(p[1], v[q] + 4);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[q][e] = elem_to_float<E>(A, base + e);
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = i0 + q * kThreads;
                if (i < ng) {
                    const int m = i / groups, grp = i - m * groups;
                    xs[(m * 2) * groups_max + grp] = make_float4(v[q][0], v[q][1], v[q][2], v[q][3]);
                    xs[(m * 2 + 1) * groups_max + grp] = make_float4(v[q][4], v[q][5], v[q][6], v[q][7]);
                }
            }
        }
        __syncthreads();
        auto compute = [&](int i0, const u32x4 (&w)[D][U][L]) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const int c = j + (i0 + d) * LPR;
                if (c < groups) {
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        if (m >= M) continue;
                        if constexpr (E == 0) {
                            const float4 xa = xs[(m * 2) * groups_max + c], xb = xs[(m * 2 + 1) * groups_max + c];
                            const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                            for (int u = 0; u < U; ++u) {
                                float wv[8];
                                widen<E>(w[d][u][0], wv);
                                if constexpr (L == 2) widen<E>(w[d][u][1], wv + 4);
#pragma unroll
                                for (int e = 0; e < 8; ++e) acc[u][m] = fmaf(xv[e], wv[e], acc[u][m]);
                            }
                        } else {
                            const u32x4 xq = xh[m * groups_max + c];
#pragma unroll
                            for (int u = 0; u < U; ++u) {
                                const u32x4 wq = w[d][u][0];
                                acc[u][m] = dot2<E>(xq.x, wq.x, acc[u][m]);
                                acc[u][m] = dot2<E>(xq.y, wq.y, acc[u][m]);
                                acc[u][m] = dot2<E>(xq.z, wq.z, acc[u][m]);
                                acc[u][m] = dot2<E>(xq.w, wq.w, acc[u][m]);
                            }
                        }
                    }
                }
            }
        };
        // Every pass issues the same loads (past the end they reload the last group, cached), so
        // the wait before a buffer's FMAs counts exactly the other buffer's loads.
        for (int i0 = 0; i0 < steps; i0 += 2 * D) {
            compute(i0, wa);
            load(i0 + 2 * D, wa);
            compute(i0 + D, wb);
            load(i0 + 3 * D, wb);
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int r = rb + u * G;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float tot = group_sum<LPR>(acc[u][m]);
            if (m < M && j == 0 && r < N) {
                float* c = C + static_cast<size_t>(m) * ldc + r;
                const float prev = beta == 0.0f ? 0.0f : (beta == 1.0f ? *c : *c * beta);
                *c = prev + alpha * tot;
            }
        }
    }
}

// One thread per output; any M, K, alignment.  C = beta*C + alpha * A * B^T.
template <int E>
__global__ void gemm_tb_plain_kernel(int M, int N, int K, float alpha, const void* __restrict__ A, int lda,
                                     const void* __restrict__ B, int ldb, float beta, float* __restrict__ C,
                                     int ldc) {
    const long long total = static_cast<long long>(M) * N;
    for (long long t = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int i = static_cast<int>(t / N), jj = static_cast<int>(t - static_cast<long long>(i) * N);
        float acc = 0.0f;
        for (int p = 0; p < K; ++p)
            acc = fmaf(elem_to_float<E>(A, static_cast<size_t>(i) * lda + p),
                       elem_to_float<E>(B, static_cast<size_t>(jj) * ldb + p), acc);
        float* c = C + static_cast<size_t>(i) * ldc + jj;
        const float prev = beta == 0.0f ? 0.0f : (beta == 1.0f ? *c : *c * beta);
        *c = prev + alpha * acc;
    }
}

// FP32 C = beta*C + alpha*op(A)*op(B) with BLAS transposes; one thread per output.
__global__ void sgemm_plain_kernel(bool ta, bool tb, int M, int N, int K, float alpha, const float* __restrict__ A,
                                   int lda, const float* __restrict__ B, int ldb, float beta, float* __restrict__ C,
                                   int ldc) {
    const long long total = static_cast<long long>(M) * N;
    for (long long t = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int i = static_cast<int>(t / N), jj = static_cast<int>(t - static_cast<long long>(i) * N);
        float acc = 0.0f;
        for (int p = 0; p < K; ++p) {
            const float a = ta ? A[static_cast<size_t>(p) * lda + i] : A[static_cast<size_t>(i) * lda + p];
            const float b = tb ? B[static_cast<size_t>(jj) * ldb + p] : B[static_cast<size_t>(p) * ldb + jj];
            acc = fmaf(a, b, acc);
        }
        float* c = C + static_cast<size_t>(i) * ldc + jj;
        const float prev = beta == 0.0f ? 0.0f : (beta == 1.0f ? *c : *c * beta);
        *c = prev + alpha * acc;
    }
}

__global__ void scale_c_kernel(float* C, int M, int N, int ldc, float beta) {
    const long long total = static_cast<long long>(M) * N;
    for (long long t = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int i = static_cast<int>(t / N), jj = static_cast<int>(t - static_cast<long long>(i) * N);
        float* c = C + static_cast<size_t>(i) * ldc + jj;
        *c = beta == 0.0f ? 0.0f : *c * beta;
    }
}

int plain_grid(long long total) { return static_cast<int>(std::max<long long>(1, std::min<long long>((total + 255) / 256, 8192))); }

template <int E, int LPR, int U, int MT>
hipError_t launch_lowp(int M, int N, int K, float alpha, const void* A, int lda, const void* B, int ldb, float beta,
                       float* C, int ldc, hipStream_t s) {
    constexpr int kRowsPerWg = 4 * (kWave / LPR) * U;
    constexpr int D = E == 0 ? 2 : 4;  // groups per lane and row in flight per buffer (two buffers)
    // A tile in LDS: at most 64 KiB (MT rows of kt floats), kt a multiple of 8.
    int kt = std::min(K, (65536 / (4 * std::max(M, 1))) / 8 * 8);
    kt = std::max(kt, 8);
    const size_t lds = static_cast<size_t>(MT) * kt * 4;
    const int grid = (N + kRowsPerWg - 1) / kRowsPerWg;
    if (const hipError_t e = allow_lds(gemv_lowp_kernel<E, LPR, U, MT, D>, lds); e != hipSuccess) return e;
    constexpr size_t es = E == 0 ? 4 : 2;
    const int a_vec = reinterpret_cast<uintptr_t>(A) % 16 == 0 && (static_cast<size_t>(lda) * es) % 16 == 0;
    hipLaunchKernelGGL((gemv_lowp_kernel<E, LPR, U, MT, D>), dim3(grid), dim3(kThreads), lds, s, M, N, K, alpha, A,
                       lda, B, ldb, beta, C, ldc, kt, a_vec);
    return hipGetLastError();
}

template <int E, int MT>
hipError_t lowp_mt(int M, int N, int K, float alpha, const void* A, int lda, const void* B, int ldb, float beta,
                   float* C, int ldc, hipStream_t s) {
    if (g_lowp_lpr) {  // diagnostics: forced lanes per row and rows per lane group
        const bool u4 = g_lowp_unroll >= 4;
        switch (g_lowp_lpr) {
            case 64: return u4 ? launch_lowp<E, 64, 4, MT>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s)
                               : launch_lowp<E, 64, 2, MT>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
            case 32: return u4 ? launch_lowp<E, 32, 4, MT>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s)
                               : launch_lowp<E, 32, 2, MT>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
            case 16: return u4 ? launch_lowp<E, 16, 4, MT>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s)
                               : launch_lowp<E, 16, 2, MT>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
            default: break;
        }
    }
    // Lanes per row from the row length in 8-element groups, two rows per lane group
    // (measured on MI355X at the Llama-3-8B shapes).
    const int groups = K / 8;
    if (groups > 512) return launch_lowp<E, 64, 2, MT>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
    if (groups >= 32) return launch_lowp<E, 32, 2, MT>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
    if (groups >= 16) return launch_lowp<E, 16, 2, MT>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
    return launch_lowp<E, 8, 2, MT>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
}

template <int E>
hipError_t gemm_tb_e(int M, int N, int K, float alpha, const void* A, int lda, const void* B, int ldb, float beta,
                     float* C, int ldc, hipStream_t s) {
    constexpr int es = E == 0 ? 4 : 2;
    const bool stream_ok = M <= 8 && K % 8 == 0 && (static_cast<long long>(ldb) * es) % 16 == 0 &&
                           reinterpret_cast<uintptr_t>(B) % 16 == 0;
    if (stream_ok) {
        if (M <= 1) return lowp_mt<E, 1>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
        if (M <= 2) return lowp_mt<E, 2>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
        if (M <= 4) return lowp_mt<E, 4>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
        return lowp_mt<E, 8>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
    }
    const long long total = static_cast<long long>(M) * N;
    hipLaunchKernelGGL(gemm_tb_plain_kernel<E>, dim3(plain_grid(total)), dim3(256), 0, s, M, N, K, alpha, A, lda, B,
                       ldb, beta, C, ldc);
    return hipGetLastError();
}

}  // namespace

void set_lowp_tuning(int lanes_per_row, int unroll) {
    g_lowp_lpr = lanes_per_row;
    g_lowp_unroll = unroll;
}

hipError_t gemm_tb(int elem, int M, int N, int K, float alpha, const void* A, int lda, const void* B, int ldb,
                   float beta, float* C, int ldc, hipStream_t s) {
    if (M <= 0 || N <= 0 || K < 0) return hipSuccess;
    if (K == 0) {
        if (beta == 1.0f) return hipSuccess;
        hipLaunchKernelGGL(scale_c_kernel, dim3(plain_grid(static_cast<long long>(M) * N)), dim3(256), 0, s, C, M, N,
                           ldc, beta);
        return hipGetLastError();
    }
    switch (elem) {
        case 0: return gemm_tb_e<0>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
        case 1: return gemm_tb_e<1>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
        case 2: return gemm_tb_e<2>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t sgemm_generic(bool trans_a, bool trans_b, int M, int N, int K, float alpha, const float* A, int lda,
                         const float* B, int ldb, float beta, float* C, int ldc, hipStream_t s) {
    if (M <= 0 || N <= 0 || K < 0) return hipSuccess;
    if (trans_b && !trans_a) return gemm_tb(0, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
    if (K == 0) return gemm_tb(0, M, N, 0, alpha, A, lda, B, ldb, beta, C, ldc, s);
    const long long total = static_cast<long long>(M) * N;
    hipLaunchKernelGGL(sgemm_plain_kernel, dim3(plain_grid(total)), dim3(256), 0, s, trans_a, trans_b, M, N, K, alpha,
                       A, lda, B, ldb, beta, C, ldc);
    return hipGetLastError();
}

}  // namespace smk
