// elementwise.hip -- SiLU, softmax rows, RMSNorm and RoPE for gfx950.
//
// SiLU follows silu_avx2.cpp:38-45: x / (1 + exp(-x)) with a correctly rounded division, and
// the denominator forced to +inf when -x > 88 (so SiLU(-inf) is NaN and very negative x give
// -0).  exp is ROCm's accurate expf (OCML, about 1 ulp), not a fast approximation: the
// reference bounds SiLU at 1e-35 + 1e-6 |ref| (activations.hpp:20-23).
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

#include <algorithm>

namespace smk {
namespace {

__global__ void silu_kernel(const float* __restrict__ in, float* __restrict__ out, long long n) {
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const float x = in[i];
        const float nx = -x;
        float d = 1.0f + expf(nx);
        if (nx > 88.0f) d = __builtin_inff();
        out[i] = x / d;
    }
}

// One wave per row; FP64 exponentials and sum as the reference's scalar softmax
// (scalar_kernels.cpp:200-222): a NaN or +inf anywhere, or every entry -inf, gives NaN.
__global__ void softmax_kernel(const float* __restrict__ in, float* __restrict__ out, int rows, int n) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;
    const float* x = in + static_cast<size_t>(row) * n;
    float* y = out + static_cast<size_t>(row) * n;
    float mx = -__builtin_inff();
    int nonfinite = 0;
    for (int i = lane; i < n; i += kWave) {
        const float v = x[i];
        nonfinite |= (v != v) || (v == __builtin_inff());
        mx = fmaxf(mx, v);
    }
    mx = group_max<kWave>(mx);
    nonfinite = group_sum_int<kWave>(nonfinite);
    if (nonfinite || mx == -__builtin_inff()) {
        for (int i = lane; i < n; i += kWave) y[i] = __builtin_nanf("");
        return;
    }
    double sum = 0.0;
    for (int i = lane; i < n; i += kWave) {
        const double e = exp(static_cast<double>(x[i]) - mx);
        y[i] = static_cast<float>(e);
        sum += e;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
    const float inv = static_cast<float>(1.0 / sum);
    for (int i = lane; i < n; i += kWave) y[i] = y[i] * inv;
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

__device__ int enumerate_leaves(int n, Node* leaves) {
    Node stack[32];
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
    Frame st[32];
    float vals[32];
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

// Fast path for chunks whose pairwise tree has every leaf at one depth D (all common model
// widths: 2048 = 16 leaves of 128, 8192 = 64 of 128, and the last chunk of 14336 = 6144 =
// 64 leaves of 96).  Leaf l (0 <= l < 2^D) is reached by following the bits of l from the
// root, left on 0.  Eight lanes per leaf hold numpy's eight interleaved accumulators,
// combined as ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) (DPP; a+b == b+a bit for bit), then the
// leaf's last len % 8 values are added in order.  Sibling subtrees are then added level by
// level: within a wave by lane exchange, across waves through LDS in the same pairing.
__device__ __forceinline__ void leaf_of(int l, int depth, int n, int& start, int& len) {
    start = 0;
    len = n;
    for (int d = depth - 1; d >= 0; --d) {
        int n2 = len / 2;
        n2 -= n2 % 8;
        if ((l >> d) & 1) {
            start += n2;
            len -= n2;
        } else {
            len = n2;
        }
    }
}

template <int kThreads>
__device__ float uniform_chunk_sum(const float* __restrict__ q, int n, int depth, float* wave_sum) {
    constexpr int kWaves = kThreads / kWave;
    const int leaves = 1 << depth;
    const int l = threadIdx.x >> 3, k = threadIdx.x & 7;
    float r = 0.0f;
    int start = 0, len = 0;
    if (l < leaves) {
        leaf_of(l, depth, n, start, len);
        const int full = len - (len % 8);
        float v = q[start + k];
        r = v * v;
        for (int i = 8 + k; i < full; i += 8) {
            v = q[start + i];
            r = r + v * v;
        }
    }
    r = r + dpp_f<kDppQuadXor1>(r);
    r = r + dpp_f<kDppQuadXor2>(r);
    r = r + dpp_f<kDppHalfMirror>(r);
    if (l < leaves) {
        for (int i = len - (len % 8); i < len; ++i) {
            const float v = q[start + i];
            r = r + v * v;
        }
    }
    // Sibling leaves: lanes xor 8, 16, 32 hold leaves l^1, l^2, l^4 of the same wave.
    for (int lv = 0; lv < 3 && (2 << lv) <= leaves; ++lv) r = r + __shfl_xor(r, 8 << lv, kWave);
    if ((threadIdx.x & (kWave - 1)) == 0) wave_sum[threadIdx.x / kWave] = r;
    __syncthreads();
    const int used = leaves >= 8 ? leaves / 8 : 1;  // waves that hold leaves
    float v[kWaves];
#pragma unroll
    for (int i = 0; i < kWaves; ++i) v[i] = wave_sum[i];
#pragma unroll
    for (int width = 1; width < kWaves; width *= 2)
#pragma unroll
        for (int i = 0; i + width < kWaves; i += 2 * width)
            if (i + width < used) v[i] = v[i] + v[i + width];
    __syncthreads();  // wave_sum is rewritten by the next chunk
    return v[0];
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

// Depth at which every leaf of numpy's pairwise tree over len values sits, or -1 when the
// leaves sit at different depths (or len < 8, where numpy sums sequentially).
int uniform_depth(int len) {
    if (len < 8) return -1;
    if (len <= 128) return 0;
    int n2 = len / 2;
    n2 -= n2 % 8;
    const int a = uniform_depth(n2), b = uniform_depth(len - n2);
    return (a >= 0 && a == b) ? a + 1 : -1;
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
            const float c = cs[i], s = sn[i];
            const float ac = a * c, bs = b * s, bc = b * c, as = a * s;
            yr[2 * i] = ac - bs;
            yr[2 * i + 1] = bc + as;
        } else {
            // x*cos + rotate_half(x)*sin, rotate_half(x) = cat(-x[half:], x[:half]).
            const float lo = xr[i], hi = xr[half + i];
            const float t0 = lo * cs[i], r0 = (-hi) * sn[i];
            const float t1 = hi * cs[half + i], r1 = lo * sn[half + i];
            yr[i] = t0 + r0;
            yr[half + i] = t1 + r1;
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
    const int per = 4;
    hipLaunchKernelGGL(softmax_kernel, dim3((rows + per - 1) / per), dim3(per * kWave), 0, s, in, out, rows, n);
    return hipGetLastError();
}

hipError_t rms_norm(const float* x, const float* w, float* y, int rows, int n, double eps, hipStream_t s) {
    if (rows <= 0 || n <= 0) return hipSuccess;
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
