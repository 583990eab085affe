// q8x.hpp -- x quantized to Q8 blocks in LDS, in the layouts the Q4_0 / Q8_0 GEMV kernels read.
//
// Plane layout (kPlanes): per row of x, four planes of uint4 indexed by pair p (blocks 2p, 2p+1):
// plane 0 holds block 2p values 0-15, plane 1 values 16-31, planes 2 and 3 the same of block
// 2p+1, so a lane reading pair p of a plane gets the 16 quants that multiply 16 W bytes.  Beside
// them: FP32 scales dx [nb] and, for the reference-order Q4_0 kernels, the chain biases
// [nb][4] (-8 times the quant sum of reference lane k's eight values of the block).
#pragma once

#include "device_common.hpp"

namespace smk {

// Destination dword of quant dword k (values 4k..4k+3) of block b.
// (The plane offset q * pairs is built from selects: a multiply-add may become v_mad_u64_u32
// with an undefined high addend half, whose register can be a pending weight load that the
// compiler then waits for.)
template <bool kPlanes>
__device__ __forceinline__ int x_dword_index(int b, int k, int pairs) {
    if (!kPlanes) return 8 * b + k;
    const int p = b >> 1;
    const int qp = ((b & 1) ? 2 * pairs : 0) + ((k & 4) ? pairs : 0);  // plane 2 * (b & 1) + (k >> 2)
    return 4 * (qp + p) + (k & 3);
}

// One quad of x (4 values of a 32-value block; 8 consecutive threads hold the block) into
// the LDS quants, bias (Q4_0: -8 * sum of the block's quants) and scale; bad[m] = 1 when the
// block holds a NaN/Inf.  All 8 threads of the block must call it together (DPP reductions).
// kChainBias (reference-order Q4_0 kernel): lds_bias gets, per block b and reference lane k
// (0..3), -8 * the sum of the quants of values {4k..4k+3} and {16+4k..16+4k+3}, at
// [m * nb * 4 + 4 * b + k].
// kGemv: q8_quad_gemv (a block with a NaN or an infinity: bad[m] = 1, its quants unspecified),
// for the GEMV kernels whose row of y is then NaN; otherwise q8_quad, whose quants are exact for
// every input (the standalone quantizer returns them).
template <bool kPlanes, bool kBias, bool kChainBias = false, bool kGemv = false>
__device__ __forceinline__ void quantize_quad(const float (&v)[4], int m, int kq, int K, uint32_t* lds_q,
                                              int* lds_bias, float* lds_dx, int* bad, bool live = true) {
    const int nb = K >> 5, pairs = nb >> 1, quads = K >> 2;
    const int b = kq >> 3, k = kq & 7;
    float d;
    int fin;
    uint32_t packed;
    if constexpr (kGemv) {
        packed = q8_quad_gemv(v, d, fin);
    } else {
        int q[4];
        packed = q8_quad(v, d, q, fin);
    }
    const int s4 = dot4(packed, 0x01010101u, 0);  // the quad's four signed quants
    const int s = kBias ? group_sum_int<8>(s4) : 0;
    int chain = 0;
    if constexpr (kChainBias) chain = -8 * (s4 + __shfl_xor(s4, 4, kWave));  // quads k and k + 4 of the block
    if (live) {
        lds_q[m * quads + x_dword_index<kPlanes>(b, k, pairs)] = packed;
        if (kChainBias && k < 4) lds_bias[(m * nb + b) * 4 + k] = chain;
        if (kBias && k == 0) lds_bias[m * nb + b] = -8 * s;
        if (k == 0) lds_dx[m * nb + b] = d;
        if (!fin) bad[m] = 1;
    }
}

// Two quads of x, k and k + 4 of block b (four consecutive threads hold the block, k = 0..3),
// into the LDS quants, biases and scale as quantize_quad stores them (for a block with a NaN or
// an infinity: bad[m] = 1 and the block's quants unspecified).  The reference lane k of the
// Q4_0 order owns exactly these two quads, so its chain bias needs no other lane.
template <bool kPlanes, bool kBias, bool kChainBias = false>
__device__ __forceinline__ void quantize_oct(const float (&va)[4], const float (&vb)[4], int m, int b, int k, int K,
                                             uint32_t* lds_q, int* lds_bias, float* lds_dx, int* bad,
                                             bool live = true) {
    const int nb = K >> 5, pairs = nb >> 1, quads = K >> 2;
    float d;
    int fin;
    uint32_t pa, pb;
    q8_oct(va, vb, d, fin, pa, pb);
    const int s8 = dot4(pa, 0x01010101u, dot4(pb, 0x01010101u, 0));  // the eight signed quants
    const int s = kBias ? group_sum_int<4>(s8) : 0;
    if (live) {
        lds_q[m * quads + x_dword_index<kPlanes>(b, k, pairs)] = pa;
        lds_q[m * quads + x_dword_index<kPlanes>(b, k + 4, pairs)] = pb;
        if (kChainBias) lds_bias[(m * nb + b) * 4 + k] = -8 * s8;
        if (kBias && k == 0) lds_bias[m * nb + b] = -8 * s;
        if (k == 0) lds_dx[m * nb + b] = d;
        if (!fin) bad[m] = 1;
    }
}

// Integer dot of one reference lane over its eight values: the block's 4 quant bytes (nibble
// pairs) against x's dword of values {4k..} (xl) and of values {16+4k..} (xh), -8 * sum(x)
// included.  Exact.
__device__ __forceinline__ int lane_dot(uint32_t q, uint32_t xl, uint32_t xh, int bias) {
    return dot4(q & 0x0f0f0f0fu, xl, dot4((q >> 4) & 0x0f0f0f0fu, xh, bias));
}

// x's Q8 data of one pair position: quants of both blocks (four planes), chain biases, scales.
struct XPair {
    uint4 q0, q1, q2, q3;
    int4 bA, bB;
    float2 d;
};

__device__ __forceinline__ XPair read_x_pair(const uint32_t* lds_q, const int* lds_cb, const float* lds_dx, int pairs,
                                             int gp) {
    const uint4* planes = reinterpret_cast<const uint4*>(lds_q);
    XPair r;
    r.q0 = planes[gp];
    r.q1 = planes[pairs + gp];
    r.q2 = planes[2 * pairs + gp];
    r.q3 = planes[3 * pairs + gp];
    r.bA = reinterpret_cast<const int4*>(lds_cb)[2 * gp];
    r.bB = reinterpret_cast<const int4*>(lds_cb)[2 * gp + 1];
    r.d = *reinterpret_cast<const float2*>(lds_dx + 2 * gp);
    return r;
}

}  // namespace smk
