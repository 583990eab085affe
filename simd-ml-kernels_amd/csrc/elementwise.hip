// elementwise.hip -- SiLU, softmax rows, RMSNorm and RoPE for gfx950.
//
// SiLU is bit-exact with the reference's SIMD tables (silu_avx2.cpp:38-45 with the exp of
// simd_math.hpp:63-117): x / (1 + exp(-x)), IEEE division, the denominator forced to +inf
// when -x > 88 (so SiLU(-inf) is NaN and very negative x give -0).
//
// Softmax rows follow softmax_row_avx2 (softmax_avx2.cpp:95-186): a NaN or +inf anywhere, or
// every entry -inf, gives a NaN row; values of full groups of 8 get e = exp(x - max) by the
// same exp, and their doubles go to eight running double sums (element i into sum i % 8, in
// order), added as s0 + s1 + ... + s7; the last n % 8 values use a double exp of (x - max)
// added in order after them; every output is then multiplied by float(1 / sum).  The double
// exp of the tail is OCML's rather than glibc's: both are within one double ulp, so the
// float results agree unless a double lands within an ulp of a float rounding boundary.
//
// RMSNorm and RoPE restate examples/llama/llama.py, where they are numpy code, and are
// bit-exact with it:
//   rms_norm (llama.py:184-187): var = mean(x*x) in float32 -- numpy's reduction: chunks of
//     8192 values (the ufunc buffer size) added in order, each chunk summed pairwise (blocks
//     of at most 128 values with 8 interleaved accumulators, halves split at multiples of
//     8) -- divided by n in float64 and rounded to float32; the scale 1/sqrt(var + eps) in
//     float64, rounded to float32; y = w * (x * scale).
//   rope (llama.py:387-396 interleaved, 169-178 half-split): a*c - b*s and b*c + a*s with
//     every product and sum rounded separately (this file is built with -ffp-contract=off).
#include "device_common.hpp"
#include "launch.hpp"
#include "pairwise_sum.hpp"

#include <algorithm>

namespace smk {
namespace {

__global__ void silu_kernel(const float* __restrict__ in, float* __restrict__ out, long long n) {
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * blockDim.x)
        out[i] = silu_ref(in[i]);
}

// One 256-thread workgroup per row, in softmax_row_avx2's order (see the top of this file).
constexpr int kSoftmaxThreads = 256;

__global__ __launch_bounds__(kSoftmaxThreads) void softmax_kernel(const float* __restrict__ in,
                                                                  float* __restrict__ out, int rows, int n) {
    __shared__ float red_f[kSoftmaxThreads / kWave];
    __shared__ int red_i[kSoftmaxThreads / kWave];
    __shared__ double lane_sum[8];
    __shared__ float inv_s;
    const int row = blockIdx.x;
    const float* x = in + static_cast<size_t>(row) * n;
    float* y = out + static_cast<size_t>(row) * n;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    constexpr int kWaves = kSoftmaxThreads / kWave;
    float mx = -__builtin_inff();
    int nonfinite = 0;
    for (int i = threadIdx.x; i < n; i += kSoftmaxThreads) {
        const float v = x[i];
        const uint32_t u = __float_as_uint(v);
        nonfinite |= (u & 0x7fffffffu) > 0x7f800000u || u == 0x7f800000u;
        mx = fmaxf(mx, v);
    }
    mx = group_max<kWave>(mx);
    nonfinite = group_sum_int<kWave>(nonfinite);
    if (lane == 0) {
        red_f[wave] = mx;
        red_i[wave] = nonfinite;
    }
    __syncthreads();
    mx = red_f[0];
    nonfinite = red_i[0];
    for (int w = 1; w < kWaves; ++w) {
        mx = fmaxf(mx, red_f[w]);
        nonfinite |= red_i[w];
    }
    if (nonfinite || __float_as_uint(mx) == 0xff800000u) {
        for (int i = threadIdx.x; i < n; i += kSoftmaxThreads) y[i] = __builtin_nanf("");
        return;
    }
    const int n8 = n - n % 8;
    for (int i = threadIdx.x; i < n; i += kSoftmaxThreads) {
        const float d = x[i] - mx;
        y[i] = i < n8 ? exp_cody_waite(d) : static_cast<float>(exp(static_cast<double>(d)));
    }
    __syncthreads();  // the e values are visible to the summing lanes
    if (threadIdx.x < 8) {
        double acc = 0.0;
        for (int i = threadIdx.x; i < n8; i += 8) acc = acc + static_cast<double>(y[i]);
        lane_sum[threadIdx.x] = acc;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = lane_sum[0];
        for (int k = 1; k < 8; ++k) t = t + lane_sum[k];
        double sum = 0.0 + t;
        for (int i = n8; i < n; ++i) sum = sum + exp(static_cast<double>(x[i] - mx));
        inv_s = static_cast<float>(1.0 / sum);
    }
    __syncthreads();
    const float inv = inv_s;
    for (int i = threadIdx.x; i < n; i += kSoftmaxThreads) y[i] = y[i] * inv;
}

// numpy's float32 pairwise sum of q[0..n) (n <= 128 leaf: 8 interleaved accumulators).
__device__ float pairwise_leaf(const float* q, int n) {
    if (n < 8) {
        float r = 0.0f;
        for (int i = 0; i < n; ++i) r = r + q[i];
        return r;
    }
    float r[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) r[k] = q[k];
    int i = 8;
    for (; i < n - (n % 8); i += 8)
#pragma unroll
        for (int k = 0; k < 8; ++k) r[k] = r[k] + q[i + k];
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) res = res + q[i];
    return res;
}

// numpy reduces a float32 vector in chunks of this many values (its ufunc buffer size).
constexpr int kSumChunk = 8192;

// The recursion of numpy's pairwise_sum, walked with an explicit stack by one thread over
// leaf sums computed in parallel: leaf (start, len) with len <= 128 for every node reached.
constexpr int kMaxLeaves = 256;  // a chunk of 8192 has at most 128 leaves

struct Node { int start, len; };

// Both walks run on one thread; their stacks sit in LDS (an array indexed at run time would be
// private memory, i.e. scratch).
__device__ int enumerate_leaves(int n, Node* leaves) {
    __shared__ Node stack[32];
    int sp = 0, cnt = 0;
    stack[sp++] = {0, n};
    while (sp > 0) {
        const Node nd = stack[--sp];
        if (nd.len <= 128) {
            leaves[cnt++] = nd;
        } else {
            int n2 = nd.len / 2;
            n2 -= n2 % 8;
            stack[sp++] = {nd.start + n2, nd.len - n2};  // right popped after left
            stack[sp++] = {nd.start, n2};
        }
    }
    return cnt;  // leaves in left-to-right order
}

// Combine leaf sums in the recursion's order: sum(node) = sum(left) + sum(right).
__device__ float combine_leaves(int n, const float* leaf_sum) {
    // Post-order evaluation with an explicit stack of pending nodes and a value stack.
    struct Frame { int start, len, state; };
    __shared__ Frame st[32];
    __shared__ float vals[32];
    int sp = 0, vp = 0, leaf = 0;
    st[sp++] = {0, n, 0};
    while (sp > 0) {
        Frame& f = st[sp - 1];
        if (f.len <= 128) {
            vals[vp++] = leaf_sum[leaf++];
            --sp;
            continue;
        }
        int n2 = f.len / 2;
        n2 -= n2 % 8;
        if (f.state == 0) {
            f.state = 1;
            st[sp++] = {f.start, n2, 0};
        } else if (f.state == 1) {
            f.state = 2;
            st[sp++] = {f.start + n2, f.len - n2, 0};
        } else {
            const float b = vals[--vp], a = vals[--vp];
            vals[vp++] = a + b;
            --sp;
        }
    }
    return vals[0];
}

__device__ __forceinline__ void rms_apply(const float* xr, const float* w, float* yr, int n, float total,
                                          double eps) {
    const float var = static_cast<float>(static_cast<double>(total) / static_cast<double>(n));
    const float scale = static_cast<float>(1.0 / sqrt(static_cast<double>(var) + eps));
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float t = xr[i] * scale;
        yr[i] = w[i] * t;
    }
}

// Any width: one workgroup of 256 threads per row of x [rows, n], chunk by chunk.
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       float* __restrict__ y, int n, double eps) {
    __shared__ float sq[kSumChunk];
    __shared__ Node leaves[kMaxLeaves];
    __shared__ float leaf_sum[kMaxLeaves];
    __shared__ int n_leaves;
    __shared__ float chunk_total;
    const float* xr = x + static_cast<size_t>(blockIdx.x) * n;
    float* yr = y + static_cast<size_t>(blockIdx.x) * n;
    float total = -0.0f;
    for (int c0 = 0; c0 < n; c0 += kSumChunk) {
        const int len = min(kSumChunk, n - c0);
        for (int i = threadIdx.x; i < len; i += blockDim.x) {
            const float v = xr[c0 + i];
            sq[i] = v * v;
        }
        if (threadIdx.x == 0) n_leaves = enumerate_leaves(len, leaves);
        __syncthreads();
        for (int l = threadIdx.x; l < n_leaves; l += blockDim.x)
            leaf_sum[l] = pairwise_leaf(sq + leaves[l].start, leaves[l].len);
        __syncthreads();
        if (threadIdx.x == 0) chunk_total = combine_leaves(len, leaf_sum);
        __syncthreads();
        total = total + chunk_total;
        __syncthreads();  // sq, leaves and chunk_total are rewritten by the next chunk
    }
    rms_apply(xr, w, yr, n, total, eps);
}

template <int kThreads>
__global__ __launch_bounds__(kThreads) void rms_norm_uniform_kernel(const float* __restrict__ x,
                                                                    const float* __restrict__ w,
                                                                    float* __restrict__ y, int n, int depth_full,
                                                                    int depth_last, double eps) {
    __shared__ float wave_sum[kThreads / kWave];
    const float* xr = x + static_cast<size_t>(blockIdx.x) * n;
    float* yr = y + static_cast<size_t>(blockIdx.x) * n;
    float total = -0.0f;
    for (int c0 = 0; c0 < n; c0 += kSumChunk) {
        const int len = min(kSumChunk, n - c0);
        total = total + uniform_chunk_sum<kThreads>(xr + c0, len, c0 + len < n ? depth_full : depth_last, wave_sum);
    }
    rms_apply(xr, w, yr, n, total, eps);
}

// Rows of 2048 (16 pairwise leaves of 128): one wave per row, x and w in registers, numpy's mean
// of squares by wave_sumsq_2048 (the same operations and order as rms_norm_uniform_kernel at
// depth 4), no LDS and no barrier.
__global__ __launch_bounds__(kWave) void rms_norm_2048_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                              float* __restrict__ y, double eps) {
    const float* xr = x + static_cast<size_t>(blockIdx.x) * 2048;
    float* yr = y + static_cast<size_t>(blockIdx.x) * 2048;
    float2 xs[16], ws[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int i = wave_sumsq_index(j);
        xs[j] = *reinterpret_cast<const float2*>(xr + i);
        ws[j] = *reinterpret_cast<const float2*>(w + i);
    }
    const float total = -0.0f + wave_sumsq_2048(xs);
    const float var = static_cast<float>(static_cast<double>(total) / 2048.0);
    const float scale = static_cast<float>(1.0 / sqrt(static_cast<double>(var) + eps));
#pragma unroll
    for (int j = 0; j < 16; ++j)
        *reinterpret_cast<float2*>(yr + wave_sumsq_index(j)) =
            make_float2(ws[j].x * (xs[j].x * scale), ws[j].y * (xs[j].y * scale));
}

// x [heads, head_dim] -> y; cos/sin [head_dim] (halves equal, as rope_cos_sin makes them).
__global__ void rope_kernel(const float* __restrict__ x, const float* __restrict__ cs, const float* __restrict__ sn,
                            float* __restrict__ y, int heads, int hd, bool interleaved) {
    const int half = hd / 2;
    const int total = heads * half;
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < total; t += gridDim.x * blockDim.x) {
        const int h = t / half, i = t - h * half;
        const float* xr = x + static_cast<size_t>(h) * hd;
        float* yr = y + static_cast<size_t>(h) * hd;
        if (interleaved) {
            const float a = xr[2 * i], b = xr[2 * i + 1];
            float o0, o1;
            rope_pair_interleaved(a, b, cs[i], sn[i], o0, o1);
            yr[2 * i] = o0;
            yr[2 * i + 1] = o1;
        } else {
            const float lo = xr[i], hi = xr[half + i];
            float o0, o1;
            rope_pair_half(lo, hi, cs[i], sn[i], cs[half + i], sn[half + i], o0, o1);
            yr[i] = o0;
            yr[half + i] = o1;
        }
    }
}

int grid_for(long long n, int threads) {
    return static_cast<int>(std::max<long long>(1, std::min<long long>((n + threads - 1) / threads, 4096)));
}

}  // namespace

hipError_t silu(const float* in, float* out, long long n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(silu_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, in, out, n);
    return hipGetLastError();
}

hipError_t softmax_rows(const float* in, float* out, int rows, int n, hipStream_t s) {
    if (rows <= 0 || n <= 0) return hipSuccess;
    hipLaunchKernelGGL(softmax_kernel, dim3(rows), dim3(kSoftmaxThreads), 0, s, in, out, rows, n);
    return hipGetLastError();
}

hipError_t rms_norm(const float* x, const float* w, float* y, int rows, int n, double eps, hipStream_t s) {
    if (rows <= 0 || n <= 0) return hipSuccess;
    if (n == 2048 && reinterpret_cast<uintptr_t>(x) % 8 == 0 && reinterpret_cast<uintptr_t>(w) % 8 == 0 &&
        reinterpret_cast<uintptr_t>(y) % 8 == 0) {
        hipLaunchKernelGGL(rms_norm_2048_kernel, dim3(rows), dim3(kWave), 0, s, x, w, y, eps);
        return hipGetLastError();
    }
    const int chunks = (n + kSumChunk - 1) / kSumChunk;
    const int depth_full = uniform_depth(std::min(n, kSumChunk));
    const int depth_last = uniform_depth(n - (chunks - 1) * kSumChunk);
    if (depth_full >= 0 && depth_last >= 0 && depth_full <= 7 && depth_last <= 7) {
        const int threads = std::max(kWave, 8 << std::max(depth_full, depth_last));  // 8 lanes per leaf
#define SMK_RMS(T)                                                                                           \
    if (threads == T) {                                                                                      \
        hipLaunchKernelGGL(rms_norm_uniform_kernel<T>, dim3(rows), dim3(T), 0, s, x, w, y, n, depth_full,  \
                           depth_last, eps);                                                                 \
        return hipGetLastError();                                                                            \
    }
        SMK_RMS(64) SMK_RMS(128) SMK_RMS(256) SMK_RMS(512) SMK_RMS(1024)
#undef SMK_RMS
    }
    hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(256), 0, s, x, w, y, n, eps);
    return hipGetLastError();
}

hipError_t rope(const float* x, const float* cos, const float* sin, float* y, int heads, int head_dim,
                bool interleaved, hipStream_t s) {
    if (heads <= 0 || head_dim <= 0) return hipSuccess;
    if (head_dim % 2) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(static_cast<long long>(heads) * head_dim / 2, 256)), dim3(256), 0, s,
                       x, cos, sin, y, heads, head_dim, interleaved);
    return hipGetLastError();
}

}  // namespace smk
