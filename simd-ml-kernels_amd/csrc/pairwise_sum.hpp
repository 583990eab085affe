// pairwise_sum.hpp -- numpy's float32 pairwise summation on a workgroup (RMSNorm's mean of
// squares), shared by the RMSNorm kernels and the GEMV prologue that normalizes x itself.
#pragma once

#include "device_common.hpp"

namespace smk {

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

// pad: leaf l's values start `pad * l` floats after their place in q (a caller that stores the
// chunk with 8 spare floats per leaf makes the eight lanes of the leaves of one wave read eight
// different groups of LDS banks; with leaves of a multiple of 64 values and no padding they all
// read the same eight banks).
template <int kThreads>
__device__ __forceinline__ float uniform_chunk_sum(const float* __restrict__ q, int n, int depth, float* wave_sum,
                                                   int pad = 0) {
    constexpr int kWaves = kThreads / kWave;
    const int leaves = 1 << depth;
    const int l = threadIdx.x >> 3, k = threadIdx.x & 7;
    float r = 0.0f;
    int start = 0, len = 0;
    if (l < leaves) {
        leaf_of(l, depth, n, start, len);
        const int full = len - (len % 8);
        q += pad * l;
        // Leaves hold at most 128 values (16 per lane): every read is issued before the sums,
        // unconditionally (a read past the leaf's full groups re-reads its first value and is
        // dropped), so that the reads are not serialized by a wait each.
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int i = 8 * j + k;
            v[j] = q[start + (i < full ? i : 0)];
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = 8 * j + k < full ? v[j] : 0.0f;
        r = v[0] * v[0];
#pragma unroll
        for (int j = 1; j < 16; ++j)
            if (8 * j + k < full) r = r + v[j] * v[j];
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
    // Sibling leaves: lanes xor 8, 16, 32 hold leaves l^1, l^2, l^4 of the same wave (xor 8 is a
    // rotation by 8 inside a 16-lane DPP row, xor 16 a swizzle inside 32 lanes).
    if (leaves >= 2) r = r + dpp_f<kDppRowRor8>(r);
    if (leaves >= 4) r = r + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(r), 0x401f));
    if (leaves >= 8) r = r + __shfl_xor(r, 32, kWave);
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


// numpy's pairwise sum of the squares of 2048 values held by one wave, with no LDS and no
// workgroup barrier.  The tree over 2048 values has 16 leaves of 128 (every split exact); leaf l
// is lanes 4l .. 4l + 3, and lane 4l + m holds accumulators 2m and 2m + 1 of the leaf's eight
// (accumulator k adds x[8j + k]^2 for j = 0 .. 15 in order, starting from x[k]^2): xs[j] =
// (x[128 l + 8 j + 2 m], x[128 l + 8 j + 2 m + 1]) -- see wave_sumsq_index.  Each lane runs its
// two chains alone; then ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) by exchanges inside the quad, and
// the leaves add level by level (lanes xor 4, 8, 16, 32: leaf l with leaf l ^ 1, then pairs of
// pairs).  Every lane returns the total.  Same operations and order as uniform_chunk_sum at
// depth 4.
__device__ __forceinline__ int wave_sumsq_index(int j) {
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    return 128 * (lane >> 2) + 8 * j + 2 * (lane & 3);
}
__device__ __forceinline__ float wave_sumsq_2048(const float2 (&xs)[16]) {
    float r0 = xs[0].x * xs[0].x, r1 = xs[0].y * xs[0].y;
#pragma unroll
    for (int j = 1; j < 16; ++j) {
        r0 = r0 + xs[j].x * xs[j].x;
        r1 = r1 + xs[j].y * xs[j].y;
    }
    float t = r0 + r1;                          // r(2m) + r(2m+1)
    t = t + __shfl_xor(t, 1, kWave);            // (r0+r1)+(r2+r3), (r4+r5)+(r6+r7)
    t = t + __shfl_xor(t, 2, kWave);            // the leaf
    t = t + __shfl_xor(t, 4, kWave);
    t = t + __shfl_xor(t, 8, kWave);
    t = t + __shfl_xor(t, 16, kWave);
    t = t + __shfl_xor(t, 32, kWave);
    return t;
}

// Depth at which every leaf of numpy's pairwise tree over len values sits, or -1 when the
// leaves sit at different depths (or len < 8, where numpy sums sequentially).
inline int uniform_depth(int len) {
    if (len < 8) return -1;
    if (len <= 128) return 0;
    int n2 = len / 2;
    n2 -= n2 % 8;
    const int a = uniform_depth(n2), b = uniform_depth(len - n2);
    return (a >= 0 && a == b) ? a + 1 : -1;
}

// The uniform tree of len values splits every node into exact halves (leaves of len >> depth
// values): every split point len / 2 at each level is a multiple of 8.
inline bool uniform_equal_leaves(int len, int depth) {
    return depth >= 0 && (depth == 0 || len % (1 << (depth + 3)) == 0);
}

}  // namespace smk
