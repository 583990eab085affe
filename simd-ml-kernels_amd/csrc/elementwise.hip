// elementwise.hip -- SiLU, softmax rows, RMSNorm and RoPE for gfx950.
//
// SiLU follows silu_avx2.cpp:38-45: x / (1 + exp(-x)) with a correctly rounded division, and
// the denominator forced to +inf when -x > 88 (so SiLU(-inf) is NaN and very negative x give
// -0).  exp is ROCm's accurate expf (OCML, about 1 ulp), not a fast approximation: the
// reference bounds SiLU at 1e-35 + 1e-6 |ref| (activations.hpp:20-23).
//
// RMSNorm and RoPE restate examples/llama/llama.py, where they are numpy code, and are
// bit-exact with it:
//   rms_norm (llama.py:184-187): var = mean(x*x) in float32 -- numpy's pairwise summation
//     (blocks of at most 128 values summed with 8 interleaved accumulators, halves split at
//     multiples of 8) -- divided by n in float64 and rounded to float32; the scale
//     1/sqrt(var + eps) in float64, rounded to float32; y = w * (x * scale).
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

// The recursion of numpy's pairwise_sum, walked with an explicit stack by one thread over
// leaf sums computed in parallel: leaf (start, len) with len <= 128 for every node reached.
constexpr int kMaxLeaves = 512;  // n <= 65536

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
__device__ float combine_leaves(int n, const Node* leaves, const float* leaf_sum) {
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
    (void)leaves;
    return vals[0];
}

// One workgroup per row of x [rows, n].
__global__ void rms_norm_kernel(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y,
                                int n, double eps) {
    extern __shared__ float sq[];           // x*x, n floats
    __shared__ Node leaves[kMaxLeaves];
    __shared__ float leaf_sum[kMaxLeaves];
    __shared__ int n_leaves;
    __shared__ float scale;
    const float* xr = x + static_cast<size_t>(blockIdx.x) * n;
    float* yr = y + static_cast<size_t>(blockIdx.x) * n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = xr[i];
        sq[i] = v * v;
    }
    if (threadIdx.x == 0) n_leaves = enumerate_leaves(n, leaves);
    __syncthreads();
    for (int l = threadIdx.x; l < n_leaves; l += blockDim.x) leaf_sum[l] = pairwise_leaf(sq + leaves[l].start, leaves[l].len);
    __syncthreads();
    if (threadIdx.x == 0) {
        const float total = combine_leaves(n, leaves, leaf_sum);
        const float var = static_cast<float>(static_cast<double>(total) / static_cast<double>(n));
        scale = static_cast<float>(1.0 / sqrt(static_cast<double>(var) + eps));
    }
    __syncthreads();
    const float s = scale;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float t = xr[i] * s;
        yr[i] = w[i] * t;
    }
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
    if (n > 128 * kMaxLeaves / 2) return hipErrorInvalidValue;
    if (const hipError_t e = allow_lds(rms_norm_kernel, static_cast<size_t>(n) * 4); e != hipSuccess) return e;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(256), static_cast<size_t>(n) * 4, s, x, w, y, n, eps);
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
