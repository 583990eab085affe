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
// A refused request is returned and also cleared from the thread's last-error state: the
// launchers report a launch's status through hipGetLastError(), which would otherwise return
// this stale error for the next, valid launch.
template <class Kernel>
inline hipError_t allow_lds(Kernel kernel, size_t bytes) {
    if (bytes <= 65536) return hipSuccess;
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) (void)hipGetLastError();
    return e;
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

// ─── cross-lane reductions ──────────────────────────────────────────────────
// Within a row of 16 lanes the partner values come through DPP (no LDS round trip):
// quad_perm [1,0,3,2] and [2,3,0,1] pair lanes inside a quad, row_half_mirror pairs the two
// quads of an 8-lane group, row_mirror the two halves of a row.  After the quad steps every
// lane of a quad holds the quad's value, so a mirror partner is as good as an xor partner.
// Across rows: ds_swizzle (xor 16 inside 32 lanes) and ds_bpermute (xor 32).
constexpr int kDppQuadXor1 = 0xB1;
constexpr int kDppQuadXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
// row_shl:n -- lane i of a 16-lane row reads lane i + n of the row (lanes past the row's end
// read 0): a halving reduction whose result is wanted in the row's first lane only.
constexpr int kDppRowShl1 = 0x101;
constexpr int kDppRowShl2 = 0x102;
constexpr int kDppRowShl4 = 0x104;
constexpr int kDppRowShl8 = 0x108;
constexpr int kDppRowRor8 = 0x128;  // row_ror:8 -- lane i of a row reads lane i ^ 8

template <int ctrl>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, ctrl, 0xf, 0xf, false);
}
template <int ctrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<ctrl>(__float_as_int(v)));
}

struct AddOp {
    template <class T>
    __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct MaxOp {
    __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

template <int width, class Op>
__device__ __forceinline__ float group_reduce_f(float v, Op op) {
    static_assert(width == 1 || width == 2 || width == 4 || width == 8 || width == 16 || width == 32 || width == 64, "");
    if constexpr (width >= 2) v = op(v, dpp_f<kDppQuadXor1>(v));
    if constexpr (width >= 4) v = op(v, dpp_f<kDppQuadXor2>(v));
    if constexpr (width >= 8) v = op(v, dpp_f<kDppHalfMirror>(v));
    if constexpr (width >= 16) v = op(v, dpp_f<kDppRowMirror>(v));
    if constexpr (width >= 32) v = op(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f)));
    if constexpr (width >= 64) v = op(v, __shfl_xor(v, 32, kWave));
    return v;
}

template <int width>
__device__ __forceinline__ int group_sum_int(int v) {
    if constexpr (width >= 2) v += dpp_i<kDppQuadXor1>(v);
    if constexpr (width >= 4) v += dpp_i<kDppQuadXor2>(v);
    if constexpr (width >= 8) v += dpp_i<kDppHalfMirror>(v);
    if constexpr (width >= 16) v += dpp_i<kDppRowMirror>(v);
    if constexpr (width >= 32) v += __builtin_amdgcn_ds_swizzle(v, 0x401f);
    if constexpr (width >= 64) v += __shfl_xor(v, 32, kWave);
    return v;
}

// Sum / max over aligned groups of `width` lanes; every lane of the group gets the result.
template <int width>
__device__ __forceinline__ float group_sum(float v) { return group_reduce_f<width>(v, AddOp{}); }
template <int width>
__device__ __forceinline__ float group_max(float v) { return group_reduce_f<width>(v, MaxOp{}); }

// Workgroup barrier that orders LDS only: it waits for this wave's LDS operations
// (lgkmcnt) but not for its outstanding global loads, which stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// Bytes 2..5 of the 8-byte pair (lo, hi): the 4 bytes that start 2 bytes into lo.
__device__ __forceinline__ uint32_t skip2(uint32_t hi, uint32_t lo) {
    return __builtin_amdgcn_alignbyte(hi, lo, 2);
}

// roundf for |v| <= 127.5: half away from zero.  v + copysign(0.5 - 2^-25, v) rounds to a value
// whose truncation is roundf(v) for every float of that range (checked exhaustively on the CPU
// against the trunc / remainder form: the sum rounds up exactly when |v| has a fraction >= 1/2),
// so it is one add, one bit select and one truncating conversion.
__device__ __forceinline__ int round_half_away(float v) {
    return static_cast<int>(v + copysignf(0.49999997f, v));
}

// The block scale of the Q8 quantizers and its inverse, as the reference rounds them (IEEE
// divisions, q8_0_scalar.cpp:52-57): d = amax / 127, id = 1 / d, id = 0 when d is 0 or 1/d
// overflows.  Division-free forms with the same results for every finite amax >= 0 (all 2^31 of
// them checked on gfx950): d is the product by RN(1/127) corrected once by a fused residual; id
// is v_rcp_f32 refined by one fused Newton step, except for a subnormal d (which v_rcp_f32
// flushes), where the division is kept.
__device__ __forceinline__ void q8_scale(float amax, float& d, float& id) {
    constexpr float c = 1.0f / 127.0f;
    const float q0 = amax * c;
    d = fmaf(fmaf(-q0, 127.0f, amax), c, q0);
    float r = __builtin_amdgcn_rcpf(d);
    r = fmaf(fmaf(-d, r, 1.0f), r, r);
    if (d < 1.17549435e-38f) r = d != 0.0f ? 1.0f / d : 0.0f;
    id = r <= 3.40282347e38f ? r : 0.0f;
}

// Q8 quants of one quad of x (values 4k..4k+3 of a 32-value block whose 8 quads sit in 8
// consecutive lanes, which call this together): quantize_row_q8_0 (q8_0_scalar.cpp:36-61)
// -- d = amax / 127 (IEEE division), id = 1 / d (0 when d is 0 or 1/d overflows float,
// q8_0_scalar.cpp:33-40, 52-58), q = round half away from zero (v * id), every product rounded on
// its own.  fin = 0 when one of the quad's values is a NaN or an infinity; such a quad keeps
// q = 0.  Returns the four quants as bytes of one dword, value 4k in the low byte.
__device__ __forceinline__ uint32_t q8_quad(const float (&v)[4], float& d, int (&q)[4], int& fin) {
    fin = finite_bits(v[0]) & finite_bits(v[1]) & finite_bits(v[2]) & finite_bits(v[3]);
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = group_max<8>(amax);
    float id;
    q8_scale(amax, d, id);
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = fin ? round_half_away(v[i] * id) : 0;
    return (static_cast<uint32_t>(q[0]) & 0xffu) | ((static_cast<uint32_t>(q[1]) & 0xffu) << 8) |
           ((static_cast<uint32_t>(q[2]) & 0xffu) << 16) | (static_cast<uint32_t>(q[3]) << 24);
}

// The low bytes of four ints as one dword, q0 in the low byte.
__device__ __forceinline__ uint32_t pack_low_bytes(int q0, int q1, int q2, int q3) {
    const uint32_t lo = __builtin_amdgcn_perm(static_cast<uint32_t>(q1), static_cast<uint32_t>(q0), 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(static_cast<uint32_t>(q3), static_cast<uint32_t>(q2), 0x04000c0cu);
    return lo | hi;
}

// q8_quad for the GEMV kernels: the same d and quants for a block of finite values (the amax as
// an unsigned maximum over |v|'s bit patterns, as q8_oct), fin = 0 for the whole block when any
// of its values is a NaN or an infinity, whose quants are then unspecified (the GEMV's row of y
// is NaN).  Returns the four quants as bytes of one dword, value 4k in the low byte.
__device__ __forceinline__ uint32_t q8_quad_gemv(const float (&v)[4], float& d, int& fin) {
    constexpr uint32_t kAbs = 0x7fffffffu;
    uint32_t m = max(max(__float_as_uint(v[0]) & kAbs, __float_as_uint(v[1]) & kAbs),
                     max(__float_as_uint(v[2]) & kAbs, __float_as_uint(v[3]) & kAbs));
    m = max(m, static_cast<uint32_t>(dpp_i<kDppQuadXor1>(static_cast<int>(m))));
    m = max(m, static_cast<uint32_t>(dpp_i<kDppQuadXor2>(static_cast<int>(m))));
    m = max(m, static_cast<uint32_t>(dpp_i<kDppHalfMirror>(static_cast<int>(m))));
    fin = m < 0x7f800000u ? 1 : 0;
    float id;
    q8_scale(__uint_as_float(m), d, id);
    return pack_low_bytes(round_half_away(v[0] * id), round_half_away(v[1] * id), round_half_away(v[2] * id),
                          round_half_away(v[3] * id));
}

// Q8 quants of two quads of x, k and k + 4 (values 4k..4k+3 and 16+4k..16+4k+3) of a
// 32-value block whose four lanes (k = 0..3) call this together: for a block of finite values
// the same d and quants as q8_quad (the block's amax is a max, exact in any order; its two
// divisions done once for eight values).  The amax is taken over the bit patterns of |v| as
// unsigned integers, which order exactly as the floats for finite values and infinity, with
// every NaN above +inf: the block is finite exactly when that maximum is below +inf's bits,
// and fin = 0 otherwise.  A non-finite block's quants are unspecified (every GEMV that uses
// this turns such a row of y into NaN).  pa / pb: the two quads' quants as bytes of one dword.
__device__ __forceinline__ void q8_oct(const float (&va)[4], const float (&vb)[4], float& d, int& fin, uint32_t& pa,
                                       uint32_t& pb) {
    constexpr uint32_t kAbs = 0x7fffffffu;
    const uint32_t ma = max(max(__float_as_uint(va[0]) & kAbs, __float_as_uint(va[1]) & kAbs),
                            max(__float_as_uint(va[2]) & kAbs, __float_as_uint(va[3]) & kAbs));
    const uint32_t mb = max(max(__float_as_uint(vb[0]) & kAbs, __float_as_uint(vb[1]) & kAbs),
                            max(__float_as_uint(vb[2]) & kAbs, __float_as_uint(vb[3]) & kAbs));
    uint32_t m = max(ma, mb);
    m = max(m, static_cast<uint32_t>(dpp_i<kDppQuadXor1>(static_cast<int>(m))));
    m = max(m, static_cast<uint32_t>(dpp_i<kDppQuadXor2>(static_cast<int>(m))));
    fin = m < 0x7f800000u ? 1 : 0;
    float id;
    q8_scale(__uint_as_float(m), d, id);
    pa = pack_low_bytes(round_half_away(va[0] * id), round_half_away(va[1] * id), round_half_away(va[2] * id),
                        round_half_away(va[3] * id));
    pb = pack_low_bytes(round_half_away(vb[0] * id), round_half_away(vb[1] * id), round_half_away(vb[2] * id),
                        round_half_away(vb[3] * id));
}

// The reference's vectorised exp (simd_math.hpp:63-117, used by its SiLU and softmax): clamp
// to +-88.3762626647949 (a NaN becomes the bound, as vminps/vmaxps return their second
// operand), k = floor(z*log2e + 0.5) with one fused multiply-add, Cody-Waite reduction
// f = z - k*ln2_hi - k*ln2_lo in two fused steps, the Cephes degree-6 polynomial by fused
// Horner steps, times 2^k assembled in the exponent field.  Same operations, same roundings:
// bit-exact with the reference's SIMD tables.
__device__ __forceinline__ float exp_cody_waite(float z) {
    const float hi = 88.3762626647949f, lo = -88.3762626647949f;
    z = z < hi ? z : hi;
    z = z > lo ? z : lo;
    const float kf = floorf(fmaf(z, 1.44269504088896341f, 0.5f));
    const int ki = static_cast<int>(kf);
    float f = fmaf(-kf, 0.693359375f, z);
    f = fmaf(-kf, -2.12194440e-4f, f);
    float p = 1.3890048347e-3f;
    p = fmaf(p, f, 8.3338161260e-3f);
    p = fmaf(p, f, 4.1666668259e-2f);
    p = fmaf(p, f, 1.6666667163e-1f);
    p = fmaf(p, f, 0.5f);
    p = fmaf(p, f, 1.0f);
    p = fmaf(p, f, 1.0f);
    return p * __uint_as_float(static_cast<uint32_t>(ki + 127) << 23);
}

// SiLU as the reference's SIMD tables compute it (silu_avx2.cpp:38-45): x / (1 + exp(-x)) with
// the exp above and an IEEE division; the denominator is +inf when -x > 88 (so the result is
// -0 there and SiLU(-inf) is NaN).
__device__ __forceinline__ float silu_ref(float x) {
    const float nx = -x;
    float d = 1.0f + exp_cody_waite(nx);
    if (nx > 88.0f) d = __builtin_inff();
    return x / d;
}

// RoPE of one pair, every product and sum rounded on its own (numpy's order):
// interleaved (llama.py:387-396): (a, b) -> (a*c - b*s, b*c + a*s);
// half split (llama.py:169-178): x*cos + rotate_half(x)*sin with rotate_half = (-hi, lo).
__device__ __forceinline__ void rope_pair_interleaved(float a, float b, float c, float s, float& o0, float& o1) {
    const float ac = a * c, bs = b * s, bc = b * c, as = a * s;
    o0 = ac - bs;
    o1 = bc + as;
}
__device__ __forceinline__ void rope_pair_half(float lo, float hi, float c_lo, float s_lo, float c_hi, float s_hi,
                                               float& o_lo, float& o_hi) {
    const float t0 = lo * c_lo, r0 = (-hi) * s_lo;
    const float t1 = hi * c_hi, r1 = lo * s_hi;
    o_lo = t0 + r0;
    o_hi = t1 + r1;
}

}  // namespace smk
