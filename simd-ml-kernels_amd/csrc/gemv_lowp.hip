// gemv_lowp.hip -- C = beta*C + alpha * A * B^T for FP32 / FP16 / BF16 B stored [N, K], for gfx950.
//
// The reference's trans_b dot path (avx2_gemm_packed.cpp:358-448, 680-732, and the scalar
// gemm_rows_tb, scalar_kernels.cpp:66-84): the M <= 8 rows of A are widened to FP32 once,
// every element of B is read once and widened in registers, FP32 fused multiply-adds.
//
// Stream kernel (rows 16-byte aligned, K a multiple of 8 elements): LPR lanes share a row of
// B and each loads 16 bytes per step (8 fp16/bf16 or 4+4 fp32 values); A is staged in LDS as
// FP32 in K tiles, in two planes of float4 so that lanes read consecutive 16-byte entries.
// Everything else (odd K, unaligned rows, M > 8) takes a plain one-thread-per-output kernel.
#include "device_common.hpp"
#include "launch.hpp"

#include <algorithm>

namespace smk {
namespace {

constexpr int kThreads = 256;

template <int E>
__device__ __forceinline__ float elem_to_float(const void* base, size_t i) {
    if constexpr (E == 0) return static_cast<const float*>(base)[i];
    else if constexpr (E == 1) return half_bits_to_float(static_cast<const uint16_t*>(base)[i]);
    else return bf16_bits_to_float(static_cast<const uint16_t*>(base)[i]);
}

// 8 consecutive elements of B widened to FP32.
template <int E>
__device__ __forceinline__ void load8(const void* row, size_t k, float (&v)[8]) {
    if constexpr (E == 0) {
        const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(row) + k);
        const f32x4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const u32x4 t = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(row) + k);
        const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (E == 1) {
                v[2 * i] = half_bits_to_float(w[i]);
                v[2 * i + 1] = half_bits_to_float(w[i] >> 16);
            } else {
                v[2 * i] = __uint_as_float(w[i] << 16);
                v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
            }
        }
    }
}

template <int E, int LPR, int U, int MT>
__global__ __launch_bounds__(kThreads) void gemv_lowp_kernel(int M, int N, int K, float alpha,
                                                             const void* __restrict__ A, int lda,
                                                             const void* __restrict__ B, int ldb, float beta,
                                                             float* __restrict__ C, int ldc, int kt) {
    constexpr int G = kWave / LPR;
    constexpr int kRowsPerWg = 4 * G * U;
    extern __shared__ __align__(16) float4 xs[];  // [MT][2][kt/8]
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int g = lane / LPR, j = lane % LPR;
    const int rb = blockIdx.x * kRowsPerWg + wave * G * U + g;
    const int groups_max = kt / 8;

    float acc[U][MT];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[u][m] = 0.0f;

    for (int k0 = 0; k0 < K; k0 += kt) {
        const int klen = min(kt, K - k0);
        const int groups = klen / 8;
        __syncthreads();
        for (int i = threadIdx.x; i < M * klen; i += blockDim.x) {
            const int m = i / klen, k = i - m * klen;
            const float v = elem_to_float<E>(A, static_cast<size_t>(m) * lda + k0 + k);
            const int grp = k >> 3, h = (k >> 2) & 1, e = k & 3;
            reinterpret_cast<float*>(xs + (m * 2 + h) * groups_max + grp)[e] = v;
        }
        __syncthreads();
        for (int c = j; c < groups; c += LPR) {
            float w[U][8];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int r = rb + u * G;
                if (r < N) {
                    const char* row = static_cast<const char*>(B) + static_cast<size_t>(r) * ldb * (E == 0 ? 4 : 2);
                    load8<E>(row, static_cast<size_t>(k0) + 8 * c, w[u]);
                }
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (m >= M) continue;
                const float4 xa = xs[(m * 2) * groups_max + c], xb = xs[(m * 2 + 1) * groups_max + c];
                const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                for (int u = 0; u < U; ++u)
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[u][m] = fmaf(xv[e], w[u][e], acc[u][m]);
            }
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
    // A tile in LDS: at most 64 KiB (MT rows of kt floats), kt a multiple of 8.
    int kt = std::min(K, (65536 / (4 * std::max(M, 1))) / 8 * 8);
    kt = std::max(kt, 8);
    const size_t lds = static_cast<size_t>(MT) * kt * 4;
    const int grid = (N + kRowsPerWg - 1) / kRowsPerWg;
    if (const hipError_t e = allow_lds(gemv_lowp_kernel<E, LPR, U, MT>, lds); e != hipSuccess) return e;
    hipLaunchKernelGGL((gemv_lowp_kernel<E, LPR, U, MT>), dim3(grid), dim3(kThreads), lds, s, M, N, K, alpha, A, lda,
                       B, ldb, beta, C, ldc, kt);
    return hipGetLastError();
}

template <int E, int MT>
hipError_t lowp_mt(int M, int N, int K, float alpha, const void* A, int lda, const void* B, int ldb, float beta,
                   float* C, int ldc, hipStream_t s) {
    // Lanes per row from the row length in 8-element groups.
    const int groups = K / 8;
    if (groups >= 64) return launch_lowp<E, 64, 4, MT>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
    if (groups >= 32) return launch_lowp<E, 32, 4, MT>(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, s);
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
