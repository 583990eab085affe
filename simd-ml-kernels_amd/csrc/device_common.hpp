// device_common.hpp -- small device helpers shared by the gfx950 kernels.
//
// Every .hip file of the library is compiled with -ffp-contract=off: each float
// operation written here is one IEEE binary32 operation unless it is an explicit
// fmaf().  That keeps the quantizers bit-exact (a contracted w*id + 8.5 truncates
// differently next to an integer) and makes every fused multiply-add visible.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace smk {

// Allow `bytes` of dynamic LDS for `kernel` (above 64 KiB a launch needs the attribute; a
// gfx950 CU has 160 KiB).
template <class Kernel>
inline hipError_t allow_lds(Kernel kernel, size_t bytes) {
    if (bytes <= 65536) return hipSuccess;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(bytes));
}

constexpr int kWave = 64;

// Native vector types (the nontemporal-load builtins need them; HIP's uint4 is a struct).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float half_bits_to_float(uint32_t h16) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(h16 & 0xffffu)));
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b16) {
    return __uint_as_float((b16 & 0xffffu) << 16);
}

__device__ __forceinline__ int finite_bits(float v) {
    return (__float_as_uint(v) & 0x7f800000u) != 0x7f800000u ? 1 : 0;
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64); every lane
// of the group gets the group's sum.
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

template <int width>
__device__ __forceinline__ int group_sum_int(int v) {
#pragma unroll
    for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

template <int width>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int off = width / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// Bytes 2..5 of the 8-byte pair (lo, hi): the 4 bytes that start 2 bytes into lo.
__device__ __forceinline__ uint32_t skip2(uint32_t hi, uint32_t lo) {
    return __builtin_amdgcn_alignbyte(hi, lo, 2);
}

// roundf for |v| <= 127.5: half away from zero (v - trunc(v) is exact).
__device__ __forceinline__ int round_half_away(float v) {
    const float t = truncf(v);
    const float r = v - t;
    return static_cast<int>(t) + (r >= 0.5f ? 1 : 0) - (r <= -0.5f ? 1 : 0);
}

}  // namespace smk
