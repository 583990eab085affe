// quantize.hip -- GGUF Q4_0 / Q8_0 weight quantization on the device, and the HBM read roof.
//
// Bit-exact with ggml's reference quantizers as the reference restates them:
//   Q8_0 (q8_0_scalar.cpp:36-111): amax = max|w|, d = amax/127, id = 1/d (0 if d = 0 or
//     1/d overflows), q = roundf(w*id) half away from zero, scale = fp16(d).
//   Q4_0 (q4_0_scalar.cpp:23-78): max = the FIRST value of largest magnitude, d = max/-8,
//     id as above, q = min(15, trunc(w*id + 8.5)) with the product and the sum rounded
//     separately (this file is built with -ffp-contract=off), byte j = q[j] | q[16+j] << 4.
// A block with a NaN/Inf, or whose scale rounds to fp16 infinity, sets *bad.
//
// Eight lanes own one 32-value block (4 values each).  The fp16 scale is rounded in integer
// arithmetic (round to nearest even, overflow to infinity), not by the conversion
// instruction, so its result does not depend on the mode register.
#include "device_common.hpp"
#include "launch.hpp"

#include <algorithm>

namespace smk {
namespace {

__device__ uint32_t f32_to_f16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;
    if (a >= 0x477ff000u) return sign | 0x7c00u;
    if (a < 0x33000000u) return sign;
    const int e = static_cast<int>(a >> 23) - 127;
    const uint32_t m = (a & 0x7fffffu) | 0x800000u;
    const int drop = e >= -14 ? 13 : 13 + (-14 - e);
    uint32_t q = m >> drop;
    const uint32_t rem = m & ((1u << drop) - 1u), half = 1u << (drop - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return sign | ((e >= -14 ? static_cast<uint32_t>(e + 14) << 10 : 0u) + q);
}

__device__ __forceinline__ void store_u16(uint8_t* p, uint32_t v) {
    *reinterpret_cast<uint16_t*>(p) = static_cast<uint16_t>(v);
}

template <int BB>
__global__ __launch_bounds__(256) void quantize_weights_kernel(long long blocks, int nb, int K,
                                                               const float* __restrict__ W,
                                                               uint8_t* __restrict__ out, int* __restrict__ bad) {
    const long long lanes = blocks * 8;
    for (long long t = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; t < ((lanes + 255) / 256) * 256;
         t += static_cast<long long>(gridDim.x) * blockDim.x) {
        const bool live = t < lanes;
        const long long blk = live ? t >> 3 : 0;
        const int k = static_cast<int>(t & 7);
        const long long row = blk / nb;
        const int b = static_cast<int>(blk - row * nb);
        const float* src = W + row * K + 32 * b + 4 * k;
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (live) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = src[i];
        }
        int fin = 1;
        float amax = 0.0f;
        int arg = 0;  // position (0..31) of the first value of largest magnitude
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            fin &= finite_bits(v[i]);
            const float a = fabsf(v[i]);
            if (a > amax) { amax = a; arg = 4 * k + i; }
        }
        // Reduce (amax, arg) over the block's 8 lanes: larger magnitude wins, ties the lower index.
#pragma unroll
        for (int off = 4; off > 0; off >>= 1) {
            const float oa = __shfl_xor(amax, off, kWave);
            const int oi = __shfl_xor(arg, off, kWave);
            if (oa > amax || (oa == amax && oi < arg)) { amax = oa; arg = oi; }
        }
        // A block whose values are all zero keeps max = +0.0 (as ggml's loop, which starts at 0).
        const int owner = arg >> 2;
        const int ai = arg & 3;
        const float mx_l = ai == 0 ? v[0] : ai == 1 ? v[1] : ai == 2 ? v[2] : v[3];
        const float mx = amax > 0.0f ? __shfl(mx_l, (static_cast<int>(threadIdx.x) & (kWave - 1) & ~7) + owner, kWave) : 0.0f;
        float d, id;
        if (BB == kQ4_0Bytes) {
            d = mx / -8.0f;
        } else {
            d = amax / 127.0f;
        }
        id = d != 0.0f ? 1.0f / d : 0.0f;
        if (!(fabsf(id) <= 3.40282347e38f)) id = 0.0f;
        const uint32_t h = f32_to_f16_rne(d);
        if (live && (!fin || (h & 0x7fffu) == 0x7c00u)) atomicOr(bad, 1);
        uint8_t* dst = out + blk * BB;
        if (BB == kQ4_0Bytes) {
            uint32_t q4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = v[i] * id;
                const float s = p + 8.5f;
                int q = fin ? static_cast<int>(s) : 8;
                q4[i] = static_cast<uint32_t>(q < 15 ? q : 15);
            }
            const uint32_t mine = q4[0] | (q4[1] << 8) | (q4[2] << 16) | (q4[3] << 24);
            const uint32_t high = __shfl_down(mine, 4, 8);  // values 16+4k.. from lane k+4
            if (live && k < 4) {
                const uint32_t bytes = mine | (high << 4);
                store_u16(dst + 2 + 4 * k, bytes & 0xffffu);
                store_u16(dst + 4 + 4 * k, bytes >> 16);
            }
        } else {
            uint32_t packed = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int q = fin ? round_half_away(v[i] * id) : 0;
                packed |= (static_cast<uint32_t>(q) & 0xffu) << (8 * i);
            }
            if (live) {
                store_u16(dst + 2 + 4 * k, packed & 0xffffu);
                store_u16(dst + 4 + 4 * k, packed >> 16);
            }
        }
        if (live && k == 0) store_u16(dst, h);
    }
}

template <bool kNT>
__device__ __forceinline__ u32x4 ld16(const u32x4* p) {
    if constexpr (kNT) return __builtin_nontemporal_load(p);
    else return *p;
}

// A pure HBM read stream: workgroup b reads its own contiguous chunk of `per_wg` 16-byte words,
// four coalesced loads of 16 KiB in flight per round; the last n16 % grid words go to the first
// workgroup.  Measured on MI355X over 2 GiB: contiguous chunks with non-temporal loads 7.19 TB/s,
// cached 5.9; a grid-stride walk (each round 8 MiB apart) 5.5-6.0.
template <bool kNT>
__global__ __launch_bounds__(1024) void read_roof_kernel(const u32x4* __restrict__ src, size_t per_wg, size_t n16,
                                                         float* __restrict__ sink) {
    constexpr int kU = 4, kT = 1024;
    uint32_t acc = 0;
    const u32x4* base = src + blockIdx.x * per_wg;
    size_t i = threadIdx.x;
    for (; i + (kU - 1) * kT < per_wg; i += kU * kT) {
        u32x4 v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) v[u] = ld16<kNT>(base + i + u * kT);
#pragma unroll
        for (int u = 0; u < kU; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < per_wg; i += kT) {
        const u32x4 a = ld16<kNT>(base + i);
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (blockIdx.x == 0)
        for (size_t r = per_wg * gridDim.x + threadIdx.x; r < n16; r += kT) {
            const u32x4 a = ld16<kNT>(src + r);
            acc ^= a.x ^ a.y ^ a.z ^ a.w;
        }
    if (acc == 0x9e3779b9u) sink[blockIdx.x] = 1.0f;  // keeps the loads; practically never taken
}

// Grid-stride copy of 16-byte words (both pointers 16-byte aligned); the last nbytes % 16
// bytes are copied one by one by the first thread.  Reads and writes exactly nbytes each, so
// it also calibrates the HBM byte counters.
__global__ __launch_bounds__(256) void copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                   size_t n16, const uint8_t* __restrict__ tail_src,
                                                   uint8_t* __restrict__ tail_dst, int tail) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
        dst[i] = a;
        dst[i + stride] = b;
        dst[i + 2 * stride] = c;
        dst[i + 3 * stride] = d;
    }
    for (; i < n16; i += stride) dst[i] = src[i];
    if (blockIdx.x == 0 && threadIdx.x == 0)
        for (int t = 0; t < tail; ++t) tail_dst[t] = tail_src[t];
}

// Exhaustive check of the x quantizer's division-free forms (q8_scale, round_half_away) against
// the IEEE forms they stand for: every finite amax >= 0 (bit patterns below 0x7f800000) through
// d = amax / 127 and id = 1 / d, and every float p with |p| <= 127.5 through roundf's trunc /
// remainder form.  counts[0] += scale mismatches, counts[1] += rounding mismatches (one
// vector atomic per thread that found any).
__global__ __launch_bounds__(256) void q8_selfcheck_kernel(unsigned* counts) {
    const uint32_t stride = gridDim.x * blockDim.x;
    unsigned bad_scale = 0, bad_round = 0;
    for (uint32_t u = blockIdx.x * blockDim.x + threadIdx.x; u < 0x7f800000u; u += stride) {
        const float amax = __uint_as_float(u);
        float d, id;
        q8_scale(amax, d, id);
        const float d_ref = amax / 127.0f;
        float id_ref = d_ref != 0.0f ? 1.0f / d_ref : 0.0f;
        if (!(id_ref <= 3.40282347e38f)) id_ref = 0.0f;
        bad_scale += (__float_as_uint(d) != __float_as_uint(d_ref)) | (__float_as_uint(id) != __float_as_uint(id_ref));
        if (u <= 0x42ff0000u) {  // |p| <= 127.5, both signs
#pragma unroll
            for (int sign = 0; sign < 2; ++sign) {
                const float p = __uint_as_float(u | (sign ? 0x80000000u : 0u));
                const float t = truncf(p), r = p - t;
                const int want = static_cast<int>(t) + (r >= 0.5f ? 1 : 0) - (r <= -0.5f ? 1 : 0);
                bad_round += round_half_away(p) != want;
            }
        }
    }
    if (bad_scale) atomicAdd(&counts[0], bad_scale);
    if (bad_round) atomicAdd(&counts[1], bad_round);
}

}  // namespace

hipError_t q8_selfcheck(unsigned* counts, hipStream_t s) {
    hipLaunchKernelGGL(q8_selfcheck_kernel, dim3(4096), dim3(256), 0, s, counts);
    return hipGetLastError();
}

hipError_t copy_bytes(void* dst, const void* src, size_t bytes, hipStream_t s) {
    if (bytes == 0) return hipSuccess;
    if ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) % 16 != 0)
        return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s);
    const size_t n16 = bytes / 16;
    const int grid = static_cast<int>(std::max<size_t>(1, std::min<size_t>((n16 + 1023) / 1024, 256 * 8)));
    const auto* s8 = static_cast<const uint8_t*>(src) + n16 * 16;
    auto* d8 = static_cast<uint8_t*>(dst) + n16 * 16;
    hipLaunchKernelGGL(copy_kernel, dim3(grid), dim3(256), 0, s, static_cast<u32x4*>(dst),
                       static_cast<const u32x4*>(src), n16, s8, d8, static_cast<int>(bytes % 16));
    return hipGetLastError();
}

hipError_t quantize_weights(int block_bytes, long long rows, int K, const float* W, uint8_t* out, int* bad,
                            hipStream_t s) {
    if (rows <= 0 || K <= 0) return hipSuccess;
    if (K % 32) return hipErrorInvalidValue;
    const int nb = K / 32;
    const long long blocks = rows * nb;
    const int grid = static_cast<int>(std::min<long long>((blocks * 8 + 255) / 256, 16384));
    if (block_bytes == kQ4_0Bytes)
        hipLaunchKernelGGL(quantize_weights_kernel<kQ4_0Bytes>, dim3(grid), dim3(256), 0, s, blocks, nb, K, W, out, bad);
    else if (block_bytes == kQ8_0Bytes)
        hipLaunchKernelGGL(quantize_weights_kernel<kQ8_0Bytes>, dim3(grid), dim3(256), 0, s, blocks, nb, K, W, out, bad);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t read_roof(const void* src, size_t bytes, float* sink, bool nontemporal, hipStream_t s) {
    const size_t n16 = bytes / 16;
    if (n16 == 0) return hipSuccess;
    // One workgroup per compute unit (256 on MI355X).
    const int grid = 256;
    const size_t per_wg = n16 / grid;
    if (nontemporal)
        hipLaunchKernelGGL(read_roof_kernel<true>, dim3(grid), dim3(1024), 0, s, static_cast<const u32x4*>(src), per_wg,
                           n16, sink);
    else
        hipLaunchKernelGGL(read_roof_kernel<false>, dim3(grid), dim3(1024), 0, s, static_cast<const u32x4*>(src),
                           per_wg, n16, sink);
    return hipGetLastError();
}

}  // namespace smk
