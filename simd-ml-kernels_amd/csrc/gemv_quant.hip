// gemv_quant.hip -- decode GEMV y = x * W^T on GGUF Q4_0 / Q8_0 blocks, for gfx950.
//
// Semantics are those of the reference's gemv_q4_0 / gemv_q8_0 (q4_0.hpp:23-33,
// q8_0.hpp:18-28, driver q8_0_scalar.cpp:120-166): x is quantized once to Q8 blocks
// (int8 quants, FP32 scales dx = amax/127), every 32-term block product is an exact
// int32, and y[n] = sum_b fp16(dw[n][b]) * dx[b] * isum[n][b] in FP32.
//
// Layout in HBM: W is read exactly as GGUF stores it, N rows of K/32 blocks (18 or 34
// bytes each), never repacked.  Two consecutive blocks form a 36- or 68-byte "pair"
// that always starts on a 4-byte boundary, so a lane streams whole pairs with 16-byte
// loads (dwordx4, 4-byte aligned) and v_alignbyte moves the block-A bytes past the
// 2-byte scale.  Each W byte is read once; x (K floats) is re-read by every workgroup
// from L2.
//
// Per workgroup (256 threads = 4 waves):
//   1. issue the first pair loads of W (so HBM latency overlaps step 2),
//   2. quantize x into LDS, bit-exact with quantize_x_q8 (q8_0_scalar.cpp:36-61,
//      308-313): IEEE amax/127 and 1/d, product and rounding as separate operations,
//      ties away from zero.  Q4_0 also stores -8 * sum(qx) per block, the starting
//      value of the block's dot so that sum((q-8)*qx) = sum(q*qx) - 8*sum(qx)
//      (the identity of q4_0_rows.hpp:25-31),
//   3. each wave walks its rows of W: LPR lanes share a row, a lane owns pairs
//      j, j+LPR, ...; v_dot4_i32_i8 does the 32-term integer sums; one fmaf per block
//      adds isum * (dw * dx) into the lane's FP32 partial; a shuffle tree sums the
//      LPR partials.  Loads for the next step are issued before the current step's
//      arithmetic (two register buffers).
//
// LDS layout of the x quants (pair kernel): four planes of uint4 per row of x,
// plane q holds, for every pair p, the 16 quants that multiply 16 W bytes of that
// pair: q=0 block 2p values 0-15, q=1 block 2p values 16-31, q=2/3 block 2p+1.
// Lanes j, j+1, ... read consecutive 16-byte entries of a plane: no bank conflicts.
#include "device_common.hpp"
#include "launch.hpp"
#include "pairwise_sum.hpp"
#include "q8x.hpp"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <type_traits>

namespace smk {
namespace {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef float f32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kThreads = 256;
// Rows of x from which a Q4_0 product takes the matrix-core kernel.  Measured on MI355X
// (graph-replayed, us, matrix-core / 8-row GEMV launches): 14336x4096 M=2 20.0/20.0, M=3
// 20.0/25.5, M=4 17.9/31.4, M=8 21.2/57.3, M=32 40.2/229; 8192x2048 M=2 ~11/9.3, M=4
// 11.2/13.6, M=32 23.7/83.3; 2048x8192 (128 row tiles for 256 CUs) M=4 30.3/28.6, M=8 33.0/193.
constexpr int kMfmaMinRows = 3;
inline bool mfma_rows_pay(int M, int N) { return M > 4 || N >= 4096; }

// The first PQ quads a thread quantizes are loaded into registers before the kernel issues
// its weight loads, so that waiting for x does not wait for W (global loads retire in
// order); quads past PQ * NT (very long rows) are loaded and quantized afterwards.
template <int NT, int PQ, int MT>
struct XPreload {
    // Units of eight values ("octs", two quads k and k + 4 of one block, quantize_oct): oct o of
    // row m is block o / 4, k = o % 4.  PQ octs a thread are loaded before the weights.
    float va[PQ][4], vb[PQ][4];
    // A wave loads pass p only when one of its lanes has an oct there (waves past the end of
    // x neither load nor quantize, and leave the SIMD to those that do).  Within a loading
    // wave the loads are unconditional (an index past the end reloads oct 0), so the wait
    // for x has a known count of younger loads and does not wait for the weights issued
    // after it.  The loads sit in blocks of their own, ahead of the weight loads: a load in
    // the same block as a wave-uniform branch to its only use is moved by the compiler into
    // that branch, behind the weights.
    __device__ __forceinline__ static bool wave_has(int p, int total) {
        return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) & ~(kWave - 1)) + p * NT < total;
    }
    __device__ __forceinline__ static const float* oct_src(const float* x, int ldx, int octs, int o) {
        const int m = MT == 1 ? 0 : o / octs, r = o - m * octs;
        return x + static_cast<size_t>(m) * ldx + 32 * (r >> 2) + 4 * (r & 3);
    }
    __device__ __forceinline__ void load(const float* __restrict__ x, int ldx, int M, int K) {
        const int octs = K >> 3, total = M * octs;
#pragma unroll
        for (int p = 0; p < PQ; ++p) {
            if (!wave_has(p, total)) break;
            int o = static_cast<int>(threadIdx.x) + p * NT;
            o = o < total ? o : 0;
            const float* src = oct_src(x, ldx, octs, o);
            const f32x4a4 a = *reinterpret_cast<const f32x4a4*>(src);
            const f32x4a4 b = *reinterpret_cast<const f32x4a4*>(src + 16);
            va[p][0] = a.x;
            va[p][1] = a.y;
            va[p][2] = a.z;
            va[p][3] = a.w;
            vb[p][0] = b.x;
            vb[p][1] = b.y;
            vb[p][2] = b.z;
            vb[p][3] = b.w;
        }
    }
    template <bool kPlanes, bool kBias, bool kChainBias = false>
    __device__ __forceinline__ void quantize(const float* __restrict__ x, int ldx, int M, int K, uint32_t* lds_q,
                                             int* lds_bias, float* lds_dx, int* bad) {
        const int octs = K >> 3, total = M * octs;
#pragma unroll
        for (int p = 0; p < PQ; ++p) {
            if (!wave_has(p, total)) break;
            const int o = static_cast<int>(threadIdx.x) + p * NT;
            const bool live = o < total;
            const int oe = live ? o : 0, m = MT == 1 ? 0 : oe / octs, r = oe - m * octs;
            quantize_oct<kPlanes, kBias, kChainBias>(va[p], vb[p], m, r >> 2, r & 3, K, lds_q, lds_bias, lds_dx, bad,
                                                     live);
        }
        for (int o = static_cast<int>(threadIdx.x) + PQ * NT; o < total; o += NT) {
            const int m = MT == 1 ? 0 : o / octs, r = o - m * octs;
            const float* src = oct_src(x, ldx, octs, o);
            const f32x4a4 a = *reinterpret_cast<const f32x4a4*>(src);
            const f32x4a4 b = *reinterpret_cast<const f32x4a4*>(src + 16);
            const float ua[4] = {a.x, a.y, a.z, a.w}, ub[4] = {b.x, b.y, b.z, b.w};
            quantize_oct<kPlanes, kBias, kChainBias>(ua, ub, m, r >> 2, r & 3, K, lds_q, lds_bias, lds_dx, bad);
        }
    }
};

// All quads of x in a strided loop (the generic and standalone kernels).
template <bool kPlanes, bool kBias>
__device__ void quantize_x_into_lds(const float* __restrict__ x, int ldx, int M, int K, uint32_t* lds_q,
                                    int* lds_bias, float* lds_dx, int* bad) {
    const int quads = K >> 2, total = M * quads;
    for (int qd = threadIdx.x; qd < total; qd += blockDim.x) {
        const int m = qd / quads, kq = qd - m * quads;
        const float* src = x + static_cast<size_t>(m) * ldx + 4 * kq;
        const float t[4] = {src[0], src[1], src[2], src[3]};
        quantize_quad<kPlanes, kBias>(t, m, kq, K, lds_q, lds_bias, lds_dx, bad);
    }
}

// ─── the pair kernel (K/32 even, W 4-byte aligned) ──────────────────────────

template <int BB>
struct PairTraits;
template <>
struct PairTraits<kQ4_0Bytes> {
    static constexpr int kDwords = 9;  // 36 bytes
    static constexpr bool kBias = true;
};
template <>
struct PairTraits<kQ8_0Bytes> {
    static constexpr int kDwords = 17;  // 68 bytes
    static constexpr bool kBias = false;
};

// Plain (cached) loads: neighbouring lanes' pairs share 128-byte lines and each line is
// touched by the two 16-byte loads and the 4-byte load of a pair, so the vector L1 must keep
// it between them (a non-temporal hint made those touches go back to L2: 11.2 -> 8.0 us at
// 14336 x 4096 without it).
template <int D>
__device__ __forceinline__ void load_pair(const uint8_t* src, uint32_t (&w)[D]) {
    const u32x4a4* v = reinterpret_cast<const u32x4a4*>(src);
#pragma unroll
    for (int i = 0; i < D / 4; ++i) {
        const u32x4a4 t = v[i];
        w[4 * i + 0] = t.x;
        w[4 * i + 1] = t.y;
        w[4 * i + 2] = t.z;
        w[4 * i + 3] = t.w;
    }
    w[D - 1] = reinterpret_cast<const uint32_t*>(src)[D - 1];
}

// Integer sums of one pair: sA for block 2p, sB for block 2p+1.  xq[0..3]: the four planes.
__device__ __forceinline__ void pair_isums(const uint32_t (&w)[9], const uint4 (&xq)[4], int biasA, int biasB,
                                           int& sA, int& sB) {
    constexpr uint32_t lo4 = 0x0f0f0f0fu;
    // Block A: scale in bytes 0-1, nibbles in bytes 2-17.
    const uint32_t a0 = skip2(w[1], w[0]), a1 = skip2(w[2], w[1]), a2 = skip2(w[3], w[2]), a3 = skip2(w[4], w[3]);
    int s = biasA;
    s = dot4(a0 & lo4, xq[0].x, s);
    s = dot4(a1 & lo4, xq[0].y, s);
    s = dot4(a2 & lo4, xq[0].z, s);
    s = dot4(a3 & lo4, xq[0].w, s);
    s = dot4((a0 >> 4) & lo4, xq[1].x, s);
    s = dot4((a1 >> 4) & lo4, xq[1].y, s);
    s = dot4((a2 >> 4) & lo4, xq[1].z, s);
    s = dot4((a3 >> 4) & lo4, xq[1].w, s);
    sA = s;
    // Block B: scale in bytes 18-19 (high half of w[4]), nibbles in w[5..8].
    s = biasB;
    s = dot4(w[5] & lo4, xq[2].x, s);
    s = dot4(w[6] & lo4, xq[2].y, s);
    s = dot4(w[7] & lo4, xq[2].z, s);
    s = dot4(w[8] & lo4, xq[2].w, s);
    s = dot4((w[5] >> 4) & lo4, xq[3].x, s);
    s = dot4((w[6] >> 4) & lo4, xq[3].y, s);
    s = dot4((w[7] >> 4) & lo4, xq[3].z, s);
    s = dot4((w[8] >> 4) & lo4, xq[3].w, s);
    sB = s;
}

__device__ __forceinline__ void pair_isums(const uint32_t (&w)[17], const uint4 (&xq)[4], int, int, int& sA,
                                           int& sB) {
    // Block A: scale bytes 0-1, quants bytes 2-33; block B: scale bytes 34-35, quants 36-67.
    int s = 0;
    s = dot4(skip2(w[1], w[0]), xq[0].x, s);
    s = dot4(skip2(w[2], w[1]), xq[0].y, s);
    s = dot4(skip2(w[3], w[2]), xq[0].z, s);
    s = dot4(skip2(w[4], w[3]), xq[0].w, s);
    s = dot4(skip2(w[5], w[4]), xq[1].x, s);
    s = dot4(skip2(w[6], w[5]), xq[1].y, s);
    s = dot4(skip2(w[7], w[6]), xq[1].z, s);
    s = dot4(skip2(w[8], w[7]), xq[1].w, s);
    sA = s;
    s = 0;
    s = dot4(w[9], xq[2].x, s);
    s = dot4(w[10], xq[2].y, s);
    s = dot4(w[11], xq[2].z, s);
    s = dot4(w[12], xq[2].w, s);
    s = dot4(w[13], xq[3].x, s);
    s = dot4(w[14], xq[3].y, s);
    s = dot4(w[15], xq[3].z, s);
    s = dot4(w[16], xq[3].w, s);
    sB = s;
}

template <int D>
__device__ __forceinline__ float scale_a(const uint32_t (&w)[D]) { return half_bits_to_float(w[0]); }
template <int D>
__device__ __forceinline__ float scale_b(const uint32_t (&w)[D]) { return half_bits_to_float(w[D / 2] >> 16); }

// BB: block bytes; LPR: lanes per row; U: rows per lane group in one step; MT: max rows of x;
// NT: threads per workgroup.
template <int BB, int LPR, int U, int MT, int NT>
__global__ __launch_bounds__(NT) void gemv_pairs_kernel(int M, int N, int K, const float* __restrict__ x, int ldx,
                                                        const uint8_t* __restrict__ W, float* __restrict__ y, int ldy,
                                                        int rows_per_wg, int accumulate) {
    using T = PairTraits<BB>;
    constexpr int D = T::kDwords;
    constexpr int G = kWave / LPR;                 // rows side by side in one wave
    constexpr int kWaves = NT / kWave;
    constexpr int kRowsPerIter = kWaves * G * U;   // rows one workgroup step covers
    // Octs (eight values) of x a thread loads before the weights: all of a row up to K = 8 * 4 * NT
    // for one row of x (octs past them load and quantize one at a time, after the weights are in
    // flight; sized for K <= 4096 this took Q8_0 4096x14336 from 14.6 to 16.4 us).
    constexpr int PQ = MT == 1 ? (NT >= 1024 ? 2 : 4)
                               : ((MT * 512 + NT - 1) / NT < 2 ? (MT * 512 + NT - 1) / NT : 2);  // octs
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ int bad[MT];

    const int nb = K >> 5, pairs = nb >> 1, quads = K >> 2;
    const size_t row_bytes = static_cast<size_t>(nb) * BB;
    uint32_t* lds_q = lds;
    int* lds_bias = reinterpret_cast<int*>(lds + M * quads);
    float* lds_dx = reinterpret_cast<float*>(lds_bias + M * nb);

    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int g = lane / LPR, j = lane % LPR;
    const int row0 = blockIdx.x * rows_per_wg;
    const int row_end = min(N, row0 + rows_per_wg);
    const int chunks = (pairs + LPR - 1) / LPR;
    const int iters = (row_end - row0 + kRowsPerIter - 1) / kRowsPerIter;
    const int steps = iters * chunks;

    if (threadIdx.x < MT) bad[threadIdx.x] = 0;
    lds_barrier();  // nothing global is in flight yet

    // Every lane loads on every step, from a clamped (valid) row and pair when its own is
    // past the end: with no load under a lane-dependent branch the compiler's wait counts
    // stay exact, so the next step's loads remain in flight while this step computes.
    auto load_step = [&](int s, uint32_t (&w)[U][D]) {
        const int it = s / chunks, c = s - it * chunks;
        const int p = min(j + c * LPR, pairs - 1);
        const int rb = row0 + it * kRowsPerIter + (wave * U) * G + g;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int r = min(rb + u * G, row_end - 1);
            load_pair<D>(W + r * row_bytes + static_cast<size_t>(p) * (2 * BB), w[u]);
        }
    };

    // x first, then the first weight step: the x-quant below waits only for x.
    XPreload<NT, PQ, MT> xp;
    xp.load(x, ldx, M, K);
    // Keep every x load ahead of the weight loads: a compiler-only fence (no instruction)
    // for the IR passes and a scheduling barrier for the machine scheduler.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_sched_barrier(0);
    // Every wave issues its x loads before any wave issues weight loads: a CU returns vector
    // loads in issue order, and x queued behind other waves' weights arrived with them.
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    uint32_t wa[U][D], wb[U][D];
    load_step(0, wa);  // steps >= 1: K/32 >= 2 and every workgroup owns at least one row
    __builtin_amdgcn_sched_barrier(0);
    xp.template quantize<true, T::kBias>(x, ldx, M, K, lds_q, lds_bias, lds_dx, bad);
    lds_barrier();  // x quants visible; the weight loads stay in flight

    float acc[U][MT];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[u][m] = 0.0f;

    auto body = [&](int s, uint32_t (&cur)[U][D], uint32_t (&nxt)[U][D]) {
        load_step(s + 1 < steps ? s + 1 : s, nxt);  // the last step reloads its own (cached) bytes
        const int it = s / chunks, c = s - it * chunks;
        const int p = j + c * LPR;
        if (p < pairs) {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (m < M) {
                    const uint4* planes = reinterpret_cast<const uint4*>(lds_q + m * quads);
                    const uint4 xq[4] = {planes[p], planes[pairs + p], planes[2 * pairs + p], planes[3 * pairs + p]};
                    const int biasA = T::kBias ? lds_bias[m * nb + 2 * p] : 0;
                    const int biasB = T::kBias ? lds_bias[m * nb + 2 * p + 1] : 0;
                    const float dxA = lds_dx[m * nb + 2 * p], dxB = lds_dx[m * nb + 2 * p + 1];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        int sA, sB;
                        pair_isums(cur[u], xq, biasA, biasB, sA, sB);
                        const float scA = scale_a(cur[u]) * dxA;
                        const float scB = scale_b(cur[u]) * dxB;
                        acc[u][m] = fmaf(static_cast<float>(sA), scA, acc[u][m]);
                        acc[u][m] = fmaf(static_cast<float>(sB), scB, acc[u][m]);
                    }
                }
            }
        }
        if (c == chunks - 1) {
            const int rb = row0 + it * kRowsPerIter + (wave * U) * G + g;
#pragma unroll
            for (int u = 0; u < U; ++u) {
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const float tot = group_sum<LPR>(acc[u][m]);
                    acc[u][m] = 0.0f;
                    const int r = rb + u * G;
                    if (m < M && j == 0 && r < row_end) {
                        float* yp = y + static_cast<size_t>(m) * ldy + r;
                        *yp = bad[m] ? __builtin_nanf("") : (accumulate ? *yp + tot : tot);
                    }
                }
            }
        }
    };

    int s = 0;
    for (; s + 1 < steps; s += 2) {
        body(s, wa, wb);
        body(s + 1, wb, wa);
    }
    if (s < steps) body(s, wa, wb);
}

// ─── Q4_0 in the reference's SIMD order (y bit-exact with its AVX2 / AVX-512 tables) ─────
// The reference's Q4_0 row loop (q4_0_rows.hpp:71-167, shared by its AVX2, AVX-VNNI and
// AVX512-VNNI units) keeps four FP32 lanes per row: lane k holds the exact integer dot of the
// block's values {4k..4k+3} and {16+4k..16+4k+3} (minus 8 times x's sum over them) and adds
// fma(float(dot), fp16(d) * dx, acc) block after block; y = (acc0 + acc2) + (acc1 + acc3).
// The last row of an odd N (q4_row_single) keeps eight lanes, the low-nibble and high-nibble
// halves apart, and sums them lane-wise first (handled by the generic kernel below, one row).
// Integer dots are exact in any order, so for the even rows:
//   phase 1 (parallel, as the pair kernel): a lane takes a 36-byte pair of one row and
//     computes, for each block and each of the four reference lanes, that lane's integer dot
//     and the block scale; they go to LDS, [row][lane][block] (chain-major);
//   phase 2 (each wave for its own rows, no workgroup barrier): four lanes per row run the
//     four FMA chains over the blocks in order, reading four blocks per 16-byte LDS load,
//     then DPP adds the lanes as the reference's horizontal sum does.
// Row stride (entries) of the phase-1 output: a multiple of 4 (16-byte reads of four blocks)
// that is 4 mod 64, so the 16-byte reads of lanes (r, k) and (r, k + 1) fall 16 bytes apart
// in the banks.
__host__ __device__ __forceinline__ int ordered_stride(int nb) { return ((nb + 63) & ~63) + 4; }

// Orders LDS accesses of one wave (writes by some lanes, then reads by others): a wave-scope
// fence around a scheduling barrier; no workgroup barrier is needed.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// N even (an odd N's last row goes to the generic kernel, which keeps q4_row_single's order).
// CH: pairs one lane takes per row (K/64 <= CH * LPR).  The weights of the next group of rows
// (CH pairs per lane) are loaded while the current group's two phases run.
// norm_w != nullptr (M == 1, K <= 8192): x is first replaced by numpy's RMSNorm of it,
// w * (x * float(1 / sqrt(mean(x*x) + eps))) (llama.py:184-187, the pairwise mean of squares
// as the RMSNorm kernel computes it; norm_depth is the depth of its uniform tree), bit for bit
// what the separate kernel would hand over.
// kStream (one row of x, CH <= 2, the G rows of a wave a multiple of 16 bytes, W 16-byte
// aligned): each wave streams the contiguous bytes of its own G rows with coalesced 16-byte
// non-temporal loads (every 128-byte line is read by one instruction, so nothing needs the
// vector L1 between loads), stages them in its own LDS region, and its lanes read their pairs
// from there; without it, a lane loads its 36-byte pairs itself (three loads that touch the
// same lines, cached).
// kNorm: norm_w is set (the fused RMSNorm prologue; a kernel of its own, so that the wait
// counts of the plain prologue are not merged with this one's).
template <int LPR, int MT, int NT, int CH, int kStream, bool kNorm>
__global__ __launch_bounds__(NT) void gemv_q4_ordered_kernel(int M, int N, int K, const float* __restrict__ x,
                                                             int ldx, const uint8_t* __restrict__ W,
                                                             float* __restrict__ y, int ldy, int rows_per_wg,
                                                             int accumulate, const float* __restrict__ norm_w,
                                                             double norm_eps, int norm_depth, int silu_pairs,
                                                             int nbuf) {
    constexpr int D = 9;
    constexpr int G = kWave / LPR;           // rows side by side in one wave (phase 1)
    constexpr int kWaves = NT / kWave;
    constexpr int kRows = kWaves * G;        // rows of one group
    constexpr int kChains = 4 * kRows * MT;  // reference lanes of a group (phase 2), at most
    constexpr int P2 = (kChains + kWave - 1) / kWave;  // waves that run them
    // Octs of x a thread loads before the weights: a row holds at most 8 * CH * LPR octs.
    constexpr int PQN = (8 * CH * LPR * MT + NT - 1) / NT;
    constexpr int PQ = PQN < 1 ? 1 : (PQN > 4 ? 4 : PQN);
    // 16-byte stream loads per lane and group: a wave's G rows hold at most 2 * CH * LPR
    // blocks each, G * 2 * CH * LPR * 18 = 2304 * CH bytes.
    constexpr int LS = (2304 / 16 * CH + kWave - 1) / kWave;
    static_assert(P2 <= kWaves, "phase 2 needs four lanes per row and row of x");
    static_assert(!kStream || (MT == 1 && CH <= 2), "streamed groups: one row of x, at most two pairs a lane");
    static_assert(!kNorm || (MT == 1 && CH <= 2), "the fused norm: one row of x, K <= 8192");
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ int bad[MT];
    __shared__ float wave_sum[NT / kWave];
    __shared__ float norm_scale;

    const int nb = K >> 5, pairs = nb >> 1, quads = K >> 2;
    const int S = ordered_stride(nb);
    const size_t row_bytes = static_cast<size_t>(nb) * kQ4_0Bytes;
    uint32_t* lds_q = lds;                                              // M * quads
    float* lds_dx = reinterpret_cast<float*>(lds + M * quads);          // M * nb
    int* lds_cb = reinterpret_cast<int*>(lds + ((M * (quads + nb) + 3) & ~3));  // M * nb * 4 lane biases
    const int x_words = ((M * (quads + nb) + 3) & ~3) + M * nb * 4;
    // nbuf (1 or 2) buffers of the phase-1 output: [M][kRows][4][S] lane dots (exact integers
    // as floats), then [M][kRows][S] block scales.
    float* const part0 = reinterpret_cast<float*>(lds + x_words);
    const int buf_floats = 5 * M * kRows * S;

    const int lane = threadIdx.x & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int g = lane / LPR, j = lane % LPR;
    const int rl = wave * G + g;             // this lane's row within the group (phase 1)
    const int row0 = blockIdx.x * rows_per_wg;
    const int row_end = min(N, row0 + rows_per_wg);
    const int iters = (row_end - row0 + kRows - 1) / kRows;

    if (threadIdx.x < MT) bad[threadIdx.x] = 0;
    lds_barrier();

    // kStream: this wave's staging region, G rows (after the x quants, the phase-1 buffers and
    // the fused norm's x).
    const int stage_words = x_words + nbuf * buf_floats + (kNorm ? K + (8 << norm_depth) : 0);
    uint8_t* const stage = reinterpret_cast<uint8_t*>(lds + stage_words) + static_cast<size_t>(wave) * G * row_bytes;
    const int stage_chunks = static_cast<int>(G * row_bytes / 16);

    typedef uint32_t PairBuf[CH][D];
    typedef u32x4 StreamBuf[LS];
    typedef std::conditional_t<kStream != 0, StreamBuf, PairBuf> WBuf;
    WBuf wa, wb;
    float ya = 0.0f, yb = 0.0f;  // streamed groups: the outputs of the groups in wa, wb

    // Phase 2 of group it runs on P2 waves, rotating with the group: chain c = 64 * (wave's
    // turn) + lane is reference lane k = c & 3 of row r = (c >> 2) % kRows against row
    // m = (c >> 2) / kRows of x; it adds the row's blocks in order, four per LDS read.
    auto turn_of = [&](int it) {
        const int t = wave - (it % kWaves) * P2 % kWaves;
        return t < 0 ? t + kWaves : t;
    };
    auto chain_of = [&](int it) { return turn_of(it) * kWave + lane; };
    // The output such a lane adds to (accumulate), read before the next group's weight loads
    // are issued, from a clamped index on every lane: its wait never waits for those loads.
    auto y_prior = [&](int it) {
        const int c = chain_of(it);
        const int m = min((c >> 2) / kRows, M - 1);
        const int row = min(row0 + it * kRows + (c >> 2) % kRows, row_end - 1);
        return y[static_cast<size_t>(m) * ldy + (silu_pairs ? row >> 1 : row)];
    };

    // Unconditional loads from a clamped row and pair (or chunk), so the compiler's wait
    // counts stay exact.  A group past the last (the prefetch of the last groups) reads the
    // first bytes of x instead, the same for every lane: one line that every workgroup has
    // just read (cached), so these loads return quickly and move no weight bytes.
    const uint8_t* const dummy = reinterpret_cast<const uint8_t*>(x);
    auto load_group = [&](int it, WBuf& w) {
        const bool live = it < iters;
        if constexpr (kStream != 0) {
            const size_t first = static_cast<size_t>(row0 + it * kRows + wave * G) * row_bytes;
            const size_t last = static_cast<size_t>(row_end) * row_bytes - 16;
#pragma unroll
            for (int u = 0; u < LS; ++u) {
                const int c = min(u * kWave + lane, stage_chunks - 1);
                const uint8_t* a = live ? W + min(first + 16 * c, last) : dummy;
                w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4a4*>(a));
            }
        } else {
            const int r = min(row0 + it * kRows + rl, row_end - 1);
            const int p0 = min(j, pairs - 1);
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int p = min(p0 + c * LPR, pairs - 1);
                load_pair<D>(live ? W + r * row_bytes + static_cast<size_t>(p) * (2 * kQ4_0Bytes) : dummy, w[c]);
            }
        }
    };
    // The first weight loads, group 0 (two groups ahead: with its output, which is read before
    // its weights, so that waiting for the weights covers it).  Group 1 follows once x is
    // quantized: issued together, the two groups delay x behind twice the traffic.
    auto first_loads = [&]() {
        if constexpr (kStream == 2) ya = y_prior(0);
        load_group(0, wa);
    };
    // The pair (c) of this lane: from the registers, or (kStream) from the wave's staging region.
    auto pair_of = [&](const WBuf& w, int c, int p, uint32_t (&out)[D]) {
        if constexpr (kStream != 0) {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(stage + g * row_bytes + static_cast<size_t>(p) * 36);
#pragma unroll
            for (int k = 0; k < D; ++k) out[k] = src[k];
        } else {
#pragma unroll
            for (int k = 0; k < D; ++k) out[k] = w[c][k];
        }
    };

    if constexpr (kNorm) {
        // x and the norm weights first (at most 4 quads a thread: K <= 16 * NT), then the first
        // weights, so that waiting for x does not wait for W.
        float* xf = part0 + nbuf * buf_floats;  // K floats
        const float4* x4 = reinterpret_cast<const float4*>(x);
        const float4* w4 = reinterpret_cast<const float4*>(norm_w);
        float4 xr[4], wr[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (u * NT >= quads) break;  // uniform: no thread has a quad this far (no idle loads)
            const int qd = static_cast<int>(threadIdx.x) + u * NT;
            const int c = qd < quads ? qd : 0;
            xr[u] = x4[c];
            wr[u] = w4[c];
        }
        // K = 2048 (16 leaves of 128): wave 0 also loads the whole of x and computes the mean of
        // squares alone (wave_sumsq_2048), so that no other wave waits for it but once, for the
        // scale; other widths go through LDS (uniform_chunk_sum).
        const bool wave_norm = K == 2048 && norm_depth == 4 && reinterpret_cast<uintptr_t>(x) % 8 == 0;
        float2 xw[16];
        if (wave_norm && wave == 0) {
#pragma unroll
            for (int j = 0; j < 16; ++j) xw[j] = *reinterpret_cast<const float2*>(x + wave_sumsq_index(j));
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_sched_barrier(0);
        // Every wave issues its x loads before any wave issues weight loads: a CU's vector loads
        // come back in the order they were issued, and x queued behind other waves' weight loads
        // arrived with the weights (measured in the decode step: ~2900 cycles later).
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        first_loads();
        __builtin_amdgcn_sched_barrier(0);
        float scale;
        if (wave_norm) {
            if (wave == 0) {
                const float total = wave_sumsq_2048(xw);
                const float var = static_cast<float>(static_cast<double>(total) / static_cast<double>(K));
                if (lane == 0) norm_scale = static_cast<float>(1.0 / sqrt(static_cast<double>(var) + norm_eps));
            }
            lds_barrier();
            scale = norm_scale;
        } else {
            // x into LDS with 8 spare floats after every leaf of the pairwise tree (leaves of
            // K >> depth values: the host checks they are equal), read back conflict-free by the sum.
            const int leaf = K >> norm_depth;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int qd = static_cast<int>(threadIdx.x) + u * NT;
                if (qd < quads) reinterpret_cast<float4*>(xf + 8 * ((4 * qd) / leaf))[qd] = xr[u];
            }
            lds_barrier();
            const float total = uniform_chunk_sum<NT>(xf, K, norm_depth, wave_sum, 8);
            const float var = static_cast<float>(static_cast<double>(total) / static_cast<double>(K));
            scale = static_cast<float>(1.0 / sqrt(static_cast<double>(var) + norm_eps));
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (u * NT >= quads) break;  // uniform: no thread has a quad this far
            const int qd = static_cast<int>(threadIdx.x) + u * NT;
            const bool live = qd < quads;
            const float h[4] = {wr[u].x * (xr[u].x * scale), wr[u].y * (xr[u].y * scale),
                                wr[u].z * (xr[u].z * scale), wr[u].w * (xr[u].w * scale)};
            quantize_quad<true, false, true, true>(h, 0, live ? qd : 0, K, lds_q, lds_cb, lds_dx, bad, live);
        }
        lds_barrier();
    } else {
        XPreload<NT, PQ, MT> xp;
        xp.load(x, ldx, M, K);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_sched_barrier(0);
        // Pair loads: every wave's x loads ahead of all weight loads, as above.  Streamed groups
        // (non-temporal, coalesced) start without that barrier (measured faster in the decode
        // step; with pair loads 2048x8192 took 5.5 -> 5.9 us without it).
        if constexpr (kStream == 0) __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        first_loads();
        __builtin_amdgcn_sched_barrier(0);
        xp.template quantize<true, false, true>(x, ldx, M, K, lds_q, lds_cb, lds_dx, bad);
        lds_barrier();
    }

    // Phase 1 of one pair: the four reference lanes' dots of both blocks, and the scales.
    auto phase1 = [&](int p, const uint32_t (&w)[D], float* part, float* scl) {
        uint32_t qa[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) qa[k] = skip2(w[k + 1], w[k]);
        const float hA = half_bits_to_float(w[0]), hB = half_bits_to_float(w[4] >> 16);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < M) {
                const uint4* planes = reinterpret_cast<const uint4*>(lds_q + m * quads);
                const uint4 x0 = planes[p], x1 = planes[pairs + p], x2 = planes[2 * pairs + p],
                            x3 = planes[3 * pairs + p];
                const int4 bA = reinterpret_cast<const int4*>(lds_cb + m * nb * 4)[2 * p];
                const int4 bB = reinterpret_cast<const int4*>(lds_cb + m * nb * 4)[2 * p + 1];
                float* pr = part + (m * kRows + rl) * 4 * S + 2 * p;
                auto dots = [&](uint32_t qa_, uint32_t xa, uint32_t xb, int ba, uint32_t qb_, uint32_t xc, uint32_t xd,
                                int bb) {
                    return make_float2(static_cast<float>(lane_dot(qa_, xa, xb, ba)),
                                       static_cast<float>(lane_dot(qb_, xc, xd, bb)));
                };
                *reinterpret_cast<float2*>(pr) = dots(qa[0], x0.x, x1.x, bA.x, w[5], x2.x, x3.x, bB.x);
                *reinterpret_cast<float2*>(pr + S) = dots(qa[1], x0.y, x1.y, bA.y, w[6], x2.y, x3.y, bB.y);
                *reinterpret_cast<float2*>(pr + 2 * S) = dots(qa[2], x0.z, x1.z, bA.z, w[7], x2.z, x3.z, bB.z);
                *reinterpret_cast<float2*>(pr + 3 * S) = dots(qa[3], x0.w, x1.w, bA.w, w[8], x2.w, x3.w, bB.w);
                const float2 d2 = *reinterpret_cast<const float2*>(lds_dx + m * nb + 2 * p);
                *reinterpret_cast<float2*>(scl + (m * kRows + rl) * S + 2 * p) = make_float2(hA * d2.x, hB * d2.y);
            }
        }
    };

    auto phase2 = [&](int it, float y_old, const float* part, const float* scl) {
        const int c = chain_of(it);
        if (turn_of(it) < P2 && c < 4 * kRows * M) {
            const int k = c & 3, r = (c >> 2) % kRows, m = (c >> 2) / kRows;
            const int row = row0 + it * kRows + r;
            const float4* pv = reinterpret_cast<const float4*>(part + ((m * kRows + r) * 4 + k) * S);
            const float4* sv = reinterpret_cast<const float4*>(scl + (m * kRows + r) * S);
            float a = 0.0f;
            const int n4 = nb >> 2;
            int q = 0;
            // Batches of 32 blocks: all 16 reads of a batch are issued before its first FMA, so
            // the chain waits for LDS once per 32 FMAs.
            for (; q + 7 < n4; q += 8) {
                float4 vv[8], ss[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    vv[i] = pv[q + i];
                    ss[i] = sv[q + i];
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    a = fmaf(vv[i].x, ss[i].x, a);
                    a = fmaf(vv[i].y, ss[i].y, a);
                    a = fmaf(vv[i].z, ss[i].z, a);
                    a = fmaf(vv[i].w, ss[i].w, a);
                }
            }
            for (; q + 1 < n4; q += 2) {
                const float4 v0 = pv[q], v1 = pv[q + 1];
                const float4 s0 = sv[q], s1 = sv[q + 1];
                a = fmaf(v0.x, s0.x, a);
                a = fmaf(v0.y, s0.y, a);
                a = fmaf(v0.z, s0.z, a);
                a = fmaf(v0.w, s0.w, a);
                a = fmaf(v1.x, s1.x, a);
                a = fmaf(v1.y, s1.y, a);
                a = fmaf(v1.z, s1.z, a);
                a = fmaf(v1.w, s1.w, a);
            }
            if (q < n4) {
                const float4 v0 = pv[q];
                const float4 s0 = sv[q];
                a = fmaf(v0.x, s0.x, a);
                a = fmaf(v0.y, s0.y, a);
                a = fmaf(v0.z, s0.z, a);
                a = fmaf(v0.w, s0.w, a);
            }
            if (nb & 2) {  // nb is even: at most two blocks left
                const float4 v0 = pv[n4];
                const float4 s0 = sv[n4];
                a = fmaf(v0.x, s0.x, a);
                a = fmaf(v0.y, s0.y, a);
            }
            a = a + dpp_f<kDppQuadXor2>(a);   // lanes k and k + 2
            a = a + dpp_f<kDppQuadXor1>(a);   // then the two pair sums
            if (silu_pairs) {
                // Rows 2n and 2n + 1 are gate_n and up_n (kRows even, rows of a group aligned):
                // y[n] = silu(gate_n) * up_n as the reference's SIMD SiLU, then one product.
                const float up = __shfl_xor(a, 4, kWave);
                if (k == 0 && (r & 1) == 0 && row < row_end)
                    y[static_cast<size_t>(m) * ldy + (row >> 1)] = bad[m] ? __builtin_nanf("") : silu_ref(a) * up;
            } else if (k == 0 && row < row_end) {
                float* yp = y + static_cast<size_t>(m) * ldy + row;
                *yp = bad[m] ? __builtin_nanf("") : (accumulate ? y_old + a : a);
            }
        }
    };

    // One group: every wave's phase 1 into the group's buffer, a workgroup barrier, phase 2
    // on P2 waves.  With two buffers the next group's phase 1 overlaps this phase 2 (the
    // barrier after it orders the reuse of this buffer); with one, a second barrier does.
    // cur holds group it (in flight or arrived), nxt group it + 1 (in flight).  Pair loads:
    // group it + 1 is issued into nxt here.  Streamed groups: group it + 1 is already in flight
    // in nxt; once cur is staged in LDS its registers take group it + 2, so two groups stay in
    // flight through both phases.
    auto body = [&](int it, WBuf& cur, WBuf& nxt, float& ycur) {
        float* part = part0 + (nbuf == 2 ? (it & 1) * buf_floats : 0);
        float* scl = part + 4 * M * kRows * S;
        float y_old;
        // This wave's rows into its staging region (its previous group's reads are done: LDS
        // operations of a wave complete in order).
        auto stage_cur = [&]() {
            if constexpr (kStream != 0) {
#pragma unroll
                for (int u = 0; u < LS; ++u) {
                    const int c = u * kWave + lane;
                    if (c < stage_chunks) *reinterpret_cast<u32x4*>(stage + 16 * c) = cur[u];
                }
            }
        };
        if constexpr (kStream == 2) {
            stage_cur();
            y_old = ycur;
            ycur = y_prior(it + 2);
            load_group(it + 2, cur);
            wave_lds_sync();
        } else if constexpr (kStream == 1) {
            y_old = y_prior(it);
            load_group(it + 1, nxt);
            stage_cur();
            wave_lds_sync();
        } else {
            y_old = y_prior(it);
            load_group(it + 1, nxt);
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int p = j + c * LPR;
            if (p < pairs) {
                uint32_t w[D];
                pair_of(cur, c, p, w);
                phase1(p, w, part, scl);
            }
        }
        lds_barrier();
        phase2(it, y_old, part, scl);
        if (nbuf == 1) lds_barrier();
    };

    if constexpr (kStream == 2) {
        yb = y_prior(1);
        load_group(1, wb);
    }
    int it = 0;
    for (; it + 1 < iters; it += 2) {
        body(it, wa, wb, ya);
        body(it + 1, wb, wa, yb);
    }
    if (it < iters) body(it, wa, wb, ya);
}

// ─── Q4_0 in the reference order over K-chunk tiles (one row of x) ──────────
// The same arithmetic as gemv_q4_ordered_kernel, organised as a stream.  A workgroup (one per
// compute unit) owns a contiguous range of rows and walks it in tiles of 16 rows x 64 blocks (a
// 2048-value chunk of K): for each group of 16 rows, its K chunks in order.  A tile is
// 16 x 1152 bytes = 1152 sixteen-byte pieces, each 16-byte aligned (K % 256 == 0); 576 threads
// (9 waves) load exactly two pieces each with non-temporal loads, TF tiles ahead in registers.
// (Measured on MI355X: aligned linear 16-byte loads stream 5.4 TB/s at 33 MB and 7.0 TB/s at
// 295 MB; the 36-byte pairs loaded by their lanes -- two 4-byte-aligned 16-byte loads and a
// dword -- only 4.1 and 5.7 TB/s.)  One workgroup barrier per tile:
//   * every thread writes its two pieces of tile t into LDS stage buffer t % 2 and issues its
//     loads of tile t + TF;
//   * waves 0-7 ("dot waves"): lane (row 2w + lane / 32, pair lane % 32) reads its 36-byte pair
//     from the stage buffer and writes the four reference lanes' exact integer dots of both
//     blocks, as floats, and the two block scales fp16(d) * dx into dot buffer t % 2.  x's
//     quants, chain biases and scales for the lane's pair position are held in registers when a
//     row has at most two chunks (K <= 4096), else read from LDS once per tile;
//   * wave 8 ("chain wave", issue priority raised): lane 4r + k runs reference lane k's FMA chain
//     of row r over tile t - 1's blocks, in block order, carried in a register from chunk to
//     chunk of the row group; after the group's last chunk, DPP adds (a0 + a2) + (a1 + a3) and
//     lane k == 0 writes y.
// Long rows advance all 64 chains of a row group together as their chunks arrive, and the FMA
// chains run beside the next tile's dots on a wave of their own.
namespace tiled {
constexpr int kRows = 16;                                  // rows of a tile: 64 chains, one wave
constexpr int kBlocks = 64;                                // blocks of a tile (2048 values of K)
constexpr int kThreads = 576;                              // 8 dot waves + 1 chain wave
constexpr int kChainWave = 8;
constexpr int kRowBytes = kBlocks * kQ4_0Bytes;            // 1152: a row's share of a tile
constexpr int kPiecesPerRow = kRowBytes / 16;              // 72
constexpr int kPieces = kRows * kPiecesPerRow;             // 1152
constexpr int kPiecesPerThread = kPieces / kThreads;       // 2
constexpr int kStride = kBlocks + 4;                       // floats per dot row (4 mod 64: no conflicts)
constexpr int kDotFloats = (4 * kRows + kRows) * kStride;  // [16][4][68] dots, then [16][68] scales
static_assert(kPieces % kThreads == 0, "whole pieces per thread");
static_assert((kThreads / kWave - 1) * kWave == kRows * kBlocks / 2, "one pair per dot lane");
}  // namespace tiled

__host__ __device__ __forceinline__ int tiled_x_words(int K) {
    const int nb = K >> 5, quads = K >> 2;
    return ((quads + nb + 3) & ~3) + nb * 4;
}

// TF: tiles in flight (register buffers); PQ: octs of x a thread loads before the weights;
// XR: chunks per row whose x data the dot lanes hold in registers (1 or 2: the row has exactly
// that many chunks; TF a multiple of XR), 0: read from LDS each tile.
// kNorm: x is replaced by RMSNorm(x) * norm_w (K = 2048, one chunk: the mean of squares by one
// wave from registers, as the row-group kernel's prologue; the same quantized image as the
// separate RMSNorm kernel followed by the plain product).
template <int TF, int PQ, int XR, bool kNorm>
__global__ __launch_bounds__(tiled::kThreads) void gemv_q4_tiled_kernel(int N, int K, const float* __restrict__ x,
                                                                        const uint8_t* __restrict__ W,
                                                                        float* __restrict__ y, int rows_per_wg,
                                                                        int accumulate, int silu_pairs,
                                                                        const float* __restrict__ norm_w,
                                                                        double norm_eps) {
    constexpr int kThreads = tiled::kThreads, kRows = tiled::kRows, kBlocks = tiled::kBlocks;
    constexpr int kRowBytes = tiled::kRowBytes, kPiecesPerRow = tiled::kPiecesPerRow, kPieces = tiled::kPieces;
    constexpr int kPiecesPerThread = tiled::kPiecesPerThread, kStride = tiled::kStride;
    constexpr int kDotFloats = tiled::kDotFloats, kChainWave = tiled::kChainWave;
    static_assert(XR == 0 || TF % XR == 0, "the chunk of an unrolled step is static");
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ int bad[1];

    const int nb = K >> 5, pairs = nb >> 1, quads = K >> 2;
    const size_t row_bytes = static_cast<size_t>(nb) * kQ4_0Bytes;
    // LDS: x quants (four planes of pairs), dx [nb], chain biases [nb][4], two stage buffers of a
    // tile's bytes, two dot buffers, and (accumulate) the prior y of the workgroup's rows.
    uint32_t* lds_q = lds;
    float* lds_dx = reinterpret_cast<float*>(lds + quads);
    int* lds_cb = reinterpret_cast<int*>(lds + ((quads + nb + 3) & ~3));
    const int x_words = tiled_x_words(K);
    uint8_t* const stage0 = reinterpret_cast<uint8_t*>(lds + x_words);
    float* const dots0 = reinterpret_cast<float*>(lds + x_words + 2 * kPieces * 4);
    float* const y_prev = dots0 + 2 * kDotFloats;

    const int tid = static_cast<int>(threadIdx.x), lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int row0 = blockIdx.x * rows_per_wg;
    const int row_end = min(N, row0 + rows_per_wg);
    const int chunks = (nb + kBlocks - 1) / kBlocks;
    const int T = ((row_end - row0 + kRows - 1) / kRows) * chunks;

    if (tid == 0) bad[0] = 0;
    if (accumulate)
        for (int i = tid; i < row_end - row0; i += kThreads) y_prev[i] = y[row0 + i];
    lds_barrier();

    // This thread's pieces: piece i = tid + u * kThreads of a tile is row i / 72, 16-byte unit
    // i % 72 of that row's chunk (a partial last chunk clamps the unit; rows past the end clamp
    // the row; both reload bytes some other piece loads).  Tiles past the last read the first
    // 16 bytes of x instead (one line every lane shares): the load count stays fixed, so the
    // compiler's waits stay exact, and no weight byte moves twice.
    int pr[kPiecesPerThread], pq[kPiecesPerThread];
#pragma unroll
    for (int u = 0; u < kPiecesPerThread; ++u) {
        const int i = tid + u * kThreads;
        pr[u] = i / kPiecesPerRow;
        pq[u] = i - pr[u] * kPiecesPerRow;
    }
    typedef u32x4 Slot[kPiecesPerThread];
    auto load_tile = [&](int t, Slot& s) {
        const bool live = t < T;
        const int tt = live ? t : 0;
        const int g = tt / chunks, c = tt - g * chunks;
        const int units = min(kBlocks, nb - c * kBlocks) * kQ4_0Bytes / 16;
#pragma unroll
        for (int u = 0; u < kPiecesPerThread; ++u) {
            const int row = min(row0 + g * kRows + pr[u], row_end - 1);
            const uint8_t* src = W + static_cast<size_t>(row) * row_bytes + static_cast<size_t>(c) * kRowBytes +
                                 16 * min(pq[u], units - 1);
            if (!live) src = reinterpret_cast<const uint8_t*>(x);
            s[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4a4*>(src));
        }
    };
    auto stage_tile = [&](int t, const Slot& s) {
        uint8_t* st = stage0 + (t & 1) * (kPieces * 16);
#pragma unroll
        for (int u = 0; u < kPiecesPerThread; ++u)
            *reinterpret_cast<u32x4*>(st + pr[u] * kRowBytes + 16 * pq[u]) = s[u];
    };

    // Phase 1 (dot waves) of tile t: the pair of this lane against x's data xp.
    const int r1 = 2 * wave + (lane >> 5), p1 = lane & 31;
    auto phase1 = [&](int t, const XPair& xp) {
        const int g = t / chunks, c = t - g * chunks;
        if (2 * p1 >= min(kBlocks, nb - c * kBlocks)) return;
        const uint32_t* src =
            reinterpret_cast<const uint32_t*>(stage0 + (t & 1) * (kPieces * 16) + r1 * kRowBytes + 36 * p1);
        uint32_t w[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) w[k] = src[k];
        uint32_t qa[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) qa[k] = skip2(w[k + 1], w[k]);
        const float hA = half_bits_to_float(w[0]), hB = half_bits_to_float(w[4] >> 16);
        float* dots = dots0 + (t & 1) * kDotFloats;
        float* pr_ = dots + (4 * r1) * kStride + 2 * p1;
        auto dots2 = [&](uint32_t qa_, uint32_t xa, uint32_t xb, int ba, uint32_t qb_, uint32_t xc, uint32_t xd, int bb) {
            return make_float2(static_cast<float>(lane_dot(qa_, xa, xb, ba)),
                               static_cast<float>(lane_dot(qb_, xc, xd, bb)));
        };
        *reinterpret_cast<float2*>(pr_) = dots2(qa[0], xp.q0.x, xp.q1.x, xp.bA.x, w[5], xp.q2.x, xp.q3.x, xp.bB.x);
        *reinterpret_cast<float2*>(pr_ + kStride) = dots2(qa[1], xp.q0.y, xp.q1.y, xp.bA.y, w[6], xp.q2.y, xp.q3.y, xp.bB.y);
        *reinterpret_cast<float2*>(pr_ + 2 * kStride) =
            dots2(qa[2], xp.q0.z, xp.q1.z, xp.bA.z, w[7], xp.q2.z, xp.q3.z, xp.bB.z);
        *reinterpret_cast<float2*>(pr_ + 3 * kStride) =
            dots2(qa[3], xp.q0.w, xp.q1.w, xp.bA.w, w[8], xp.q2.w, xp.q3.w, xp.bB.w);
        *reinterpret_cast<float2*>(dots + (4 * kRows + r1) * kStride + 2 * p1) = make_float2(hA * xp.d.x, hB * xp.d.y);
    };

    // Phase 2 (chain wave) of tile t: the chains of its row group over its blocks.
    float acc = 0.0f;
    auto phase2 = [&](int t) {
        const int g = t / chunks, c = t - g * chunks;
        const int cn = min(kBlocks, nb - c * kBlocks);  // a multiple of 8
        const int r = lane >> 2, k = lane & 3;
        const float* dots = dots0 + (t & 1) * kDotFloats;
        const float4* pv = reinterpret_cast<const float4*>(dots + (4 * r + k) * kStride);
        const float4* sv = reinterpret_cast<const float4*>(dots + (4 * kRows + r) * kStride);
        float a = c == 0 ? 0.0f : acc;
        int q = 0;
        const int n4 = cn >> 2;
        for (; q + 7 < n4; q += 8) {  // 32 blocks a batch: 16 reads issued before the first FMA
            float4 vv[8], ss[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                vv[i] = pv[q + i];
                ss[i] = sv[q + i];
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                a = fmaf(vv[i].x, ss[i].x, a);
                a = fmaf(vv[i].y, ss[i].y, a);
                a = fmaf(vv[i].z, ss[i].z, a);
                a = fmaf(vv[i].w, ss[i].w, a);
            }
        }
        for (; q + 1 < n4; q += 2) {  // cn % 8 == 0: whole pairs of float4
            const float4 v0 = pv[q], v1 = pv[q + 1], s0 = sv[q], s1 = sv[q + 1];
            a = fmaf(v0.x, s0.x, a);
            a = fmaf(v0.y, s0.y, a);
            a = fmaf(v0.z, s0.z, a);
            a = fmaf(v0.w, s0.w, a);
            a = fmaf(v1.x, s1.x, a);
            a = fmaf(v1.y, s1.y, a);
            a = fmaf(v1.z, s1.z, a);
            a = fmaf(v1.w, s1.w, a);
        }
        acc = a;
        if (c == chunks - 1) {
            a = a + dpp_f<kDppQuadXor2>(a);  // lanes k and k + 2
            a = a + dpp_f<kDppQuadXor1>(a);  // then the two pair sums
            const int lr = g * kRows + r, row = row0 + lr;
            if (silu_pairs) {
                // Rows 2n and 2n + 1 are gate_n and up_n (row0 and kRows even): y[n] = silu(gate) * up.
                const float up = __shfl_xor(a, 4, kWave);
                if (k == 0 && (r & 1) == 0 && row < row_end) y[row >> 1] = bad[0] ? __builtin_nanf("") : silu_ref(a) * up;
            } else if (k == 0 && row < row_end) {
                y[row] = bad[0] ? __builtin_nanf("") : (accumulate ? y_prev[lr] + a : a);
            }
        }
    };

    // x first (its own loads, every wave's ahead of any weight load), then the first TF tiles,
    // then x is quantized while they are in flight.
    Slot ring[TF];
    if constexpr (kNorm) {
        static_assert(XR == 1, "the fused norm: K = 2048, one chunk");
        __shared__ float norm_scale;
        const int quads = K >> 2;  // 512 <= kThreads: one quad a thread
        const int qd = tid < quads ? tid : 0;
        const float4 xq = reinterpret_cast<const float4*>(x)[qd];
        const float4 wq = reinterpret_cast<const float4*>(norm_w)[qd];
        float2 xw[16];
        if (wave == 0) {
#pragma unroll
            for (int j = 0; j < 16; ++j) xw[j] = *reinterpret_cast<const float2*>(x + wave_sumsq_index(j));
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < TF; ++s) load_tile(s, ring[s]);
        __builtin_amdgcn_sched_barrier(0);
        if (wave == 0) {
            const float total = wave_sumsq_2048(xw);
            const float var = static_cast<float>(static_cast<double>(total) / static_cast<double>(K));
            if (lane == 0) norm_scale = static_cast<float>(1.0 / sqrt(static_cast<double>(var) + norm_eps));
        }
        lds_barrier();
        const float scale = norm_scale;
        const float h[4] = {wq.x * (xq.x * scale), wq.y * (xq.y * scale), wq.z * (xq.z * scale),
                            wq.w * (xq.w * scale)};
        quantize_quad<true, false, true, true>(h, 0, qd, K, lds_q, lds_cb, lds_dx, bad, tid < quads);
    } else {
        XPreload<kThreads, PQ, 1> xpre;
        xpre.load(x, K, 1, K);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < TF; ++s) load_tile(s, ring[s]);
        __builtin_amdgcn_sched_barrier(0);
        xpre.template quantize<true, false, true>(x, K, 1, K, lds_q, lds_cb, lds_dx, bad);
    }
    lds_barrier();
    // The dot lanes' x data, for the chunks a row has (held in registers when XR > 0).
    constexpr int kXr = XR > 0 ? XR : 1;
    XPair xr[kXr];
    if (XR > 0 && wave != kChainWave) {
#pragma unroll
        for (int c = 0; c < kXr; ++c) xr[c] = read_x_pair(lds_q, lds_cb, lds_dx, pairs, min(c * 32 + p1, pairs - 1));
    }
    // The chain wave's FMA chains are the critical path of a step (each FMA waits for the one
    // before it): it takes issue priority over the dot waves that share its SIMD.
    if (wave == kChainWave) __builtin_amdgcn_s_setprio(3);

    // Step t: stage tile t and issue tile t + TF's loads; barrier; phase 1 of tile t (dot waves)
    // beside phase 2 of tile t - 1 (chain wave).
    const int steps = (T + 1 + TF - 1) / TF * TF;  // every tile's phase 2 runs inside the loop
    for (int t0 = 0; t0 < steps; t0 += TF) {
#pragma unroll
        for (int s = 0; s < TF; ++s) {
            const int t = t0 + s;
            if (t < T) stage_tile(t, ring[s]);
            load_tile(t + TF, ring[s]);
            lds_barrier();
            if (wave == kChainWave) {
                if (t >= 1 && t - 1 < T) phase2(t - 1);
            } else if (t < T) {
                if constexpr (XR > 0) {
                    phase1(t, xr[s % kXr]);  // t0 is a multiple of TF, so chunk(t) = s % XR
                } else {
                    const int c = t % chunks;
                    phase1(t, read_x_pair(lds_q, lds_cb, lds_dx, pairs, min(c * 32 + p1, pairs - 1)));
                }
            }
        }
    }
}

// Odd K/32 or a 2-byte aligned W: four lanes per row walk the blocks themselves (16-bit
// loads), in the same order; 64 rows per 256-thread workgroup.
template <int MT>
__global__ __launch_bounds__(kThreads) void gemv_q4_ordered_generic_kernel(int M, int N, int K,
                                                                           const float* __restrict__ x, int ldx,
                                                                           const uint8_t* __restrict__ W,
                                                                           float* __restrict__ y, int ldy,
                                                                           int accumulate) {
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ int bad[MT];
    const int nb = K >> 5, quads = K >> 2;
    uint32_t* lds_q = lds;
    float* lds_dx = reinterpret_cast<float*>(lds + M * quads);
    if (threadIdx.x < MT) bad[threadIdx.x] = 0;
    lds_barrier();
    quantize_x_into_lds<false, false>(x, ldx, M, K, lds_q, nullptr, lds_dx, bad);
    lds_barrier();
    const int r = threadIdx.x >> 2, k = threadIdx.x & 3;
    const int row = blockIdx.x * (kThreads / 4) + r;
    const int rr = min(row, N - 1);
    const bool single = (N & 1) && row == N - 1;
    float a1[MT], a2[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) a1[m] = a2[m] = 0.0f;
    const uint8_t* wrow = W + static_cast<size_t>(rr) * nb * kQ4_0Bytes;
    for (int b = 0; b < nb; ++b) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(wrow + static_cast<size_t>(b) * kQ4_0Bytes);
        const uint32_t q = static_cast<uint32_t>(h[1 + 2 * k]) | (static_cast<uint32_t>(h[2 + 2 * k]) << 16);
        const float hd = half_bits_to_float(h[0]);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m >= M) break;
            const uint32_t* xb = lds_q + m * quads + 8 * b;
            constexpr uint32_t kMinus8 = 0xF8F8F8F8u;
            const int dl = dot4(q & 0x0f0f0f0fu, xb[k], dot4(kMinus8, xb[k], 0));
            const int dh = dot4((q >> 4) & 0x0f0f0f0fu, xb[4 + k], dot4(kMinus8, xb[4 + k], 0));
            const float s = hd * lds_dx[m * nb + b];
            a1[m] = fmaf(static_cast<float>(single ? dl : dl + dh), s, a1[m]);
            a2[m] = fmaf(static_cast<float>(dh), s, a2[m]);
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (m >= M) break;
        float tt = single ? a1[m] + a2[m] : a1[m];
        tt = tt + dpp_f<kDppQuadXor2>(tt);
        tt = tt + dpp_f<kDppQuadXor1>(tt);
        if (k == 0 && row < N) {
            float* yp = y + static_cast<size_t>(m) * ldy + row;
            *yp = bad[m] ? __builtin_nanf("") : (accumulate ? *yp + tt : tt);
        }
    }
}

// ─── the generic kernel (any K/32, W 2-byte aligned) ─────────────────────────
// One wave per row, lanes over blocks; 16-bit loads.  Used for odd K/32 only.
template <int BB, int MT>
__global__ __launch_bounds__(kThreads) void gemv_generic_kernel(int M, int N, int K, const float* __restrict__ x,
                                                                int ldx, const uint8_t* __restrict__ W,
                                                                float* __restrict__ y, int ldy, int rows_per_wg,
                                                                int accumulate) {
    constexpr bool kQ4 = BB == kQ4_0Bytes;
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ int bad[MT];
    const int nb = K >> 5, quads = K >> 2;
    uint32_t* lds_q = lds;
    int* lds_bias = reinterpret_cast<int*>(lds + M * quads);
    float* lds_dx = reinterpret_cast<float*>(lds_bias + M * nb);
    if (threadIdx.x < MT) bad[threadIdx.x] = 0;
    lds_barrier();
    quantize_x_into_lds<false, kQ4>(x, ldx, M, K, lds_q, lds_bias, lds_dx, bad);
    lds_barrier();

    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int row0 = blockIdx.x * rows_per_wg;
    const int row_end = min(N, row0 + rows_per_wg);
    for (int r = row0 + wave; r < row_end; r += kThreads / kWave) {
        float acc[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
        for (int b = lane; b < nb; b += kWave) {
            const uint16_t* h = reinterpret_cast<const uint16_t*>(W + (static_cast<size_t>(r) * nb + b) * BB);
            const float dw = half_bits_to_float(h[0]);
            uint32_t q[8];
#pragma unroll
            for (int k = 0; k < (kQ4 ? 4 : 8); ++k)
                q[k] = static_cast<uint32_t>(h[1 + 2 * k]) | (static_cast<uint32_t>(h[2 + 2 * k]) << 16);
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if (m >= M) continue;
                const uint32_t* xq = lds_q + m * quads + 8 * b;
                int s = kQ4 ? lds_bias[m * nb + b] : 0;
                if (kQ4) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        s = dot4(q[k] & 0x0f0f0f0fu, xq[k], s);
                        s = dot4((q[k] >> 4) & 0x0f0f0f0fu, xq[4 + k], s);
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < 8; ++k) s = dot4(q[k], xq[k], s);
                }
                acc[m] = fmaf(static_cast<float>(s), dw * lds_dx[m * nb + b], acc[m]);
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float tot = group_sum<kWave>(acc[m]);
            if (m < M && lane == 0) {
                float* yp = y + static_cast<size_t>(m) * ldy + r;
                *yp = bad[m] ? __builtin_nanf("") : (accumulate ? *yp + tot : tot);
            }
        }
    }
}

__global__ void fill_kernel(float* y, long long n, float v) {
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * blockDim.x)
        y[i] = v;
}

// ─── standalone x quantization and block sums (parity entry points) ─────────

__global__ __launch_bounds__(kThreads) void quantize_x_kernel(int K, const float* __restrict__ x,
                                                              int8_t* __restrict__ qs, float* __restrict__ dx,
                                                              int* __restrict__ bad) {
    // One workgroup per 32 blocks: reuse the LDS routine on a slice of x, then copy out.
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ int bad1[1];
    const int nb_all = K >> 5;
    const int b0 = blockIdx.x * 32;
    const int nbk = min(32, nb_all - b0);
    const int Kk = nbk * 32;
    if (threadIdx.x == 0) bad1[0] = 0;
    __syncthreads();
    int* lds_bias = reinterpret_cast<int*>(lds + (Kk >> 2));
    float* lds_dx = reinterpret_cast<float*>(lds_bias + nbk);
    quantize_x_into_lds<false, false>(x + 32 * b0, Kk, 1, Kk, lds, lds_bias, lds_dx, bad1);
    __syncthreads();
    for (int i = threadIdx.x; i < (Kk >> 2); i += blockDim.x)
        reinterpret_cast<uint32_t*>(qs + 32 * b0)[i] = lds[i];
    for (int i = threadIdx.x; i < nbk; i += blockDim.x) dx[b0 + i] = lds_dx[i];
    if (threadIdx.x == 0 && bad1[0]) atomicOr(bad, 1);
}

template <int BB>
__global__ void block_sums_kernel(int N, int K, const int8_t* __restrict__ qs, const uint8_t* __restrict__ W,
                                  int32_t* __restrict__ out) {
    const int nb = K >> 5;
    const long long total = static_cast<long long>(N) * nb;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int b = static_cast<int>(i % nb);
        const uint8_t* blk = W + i * BB + 2;
        const int8_t* xq = qs + 32 * b;
        int s = 0;
        if (BB == kQ4_0Bytes) {
            for (int t = 0; t < 16; ++t)
                s += (static_cast<int>(blk[t] & 0x0f) - 8) * xq[t] + (static_cast<int>(blk[t] >> 4) - 8) * xq[16 + t];
        } else {
            for (int t = 0; t < 32; ++t) s += static_cast<int>(static_cast<int8_t>(blk[t])) * xq[t];
        }
        out[i] = s;
    }
}

// ─── host side ───────────────────────────────────────────────────────────────

// Compute units of the device in use (set by the runtime at initialisation).
std::atomic<int> g_cus{256};

bool pair_path_ok(int K, const uint8_t* W) {
    return ((K >> 5) % 2 == 0) && (reinterpret_cast<uintptr_t>(W) % 4 == 0);
}

int choose_lpr(int pairs) {
    for (int l : {64, 32, 16, 8})
        if (pairs % l == 0) return l;
    int l = 8;
    while (l < 64 && l * 2 <= pairs) l *= 2;
    return l;
}

template <int BB, int LPR, int U, int MT, int NT>
hipError_t launch_pairs(int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y, int ldy,
                        int rows_per_wg, int acc, hipStream_t stream) {
    constexpr int G = kWave / LPR;
    constexpr int kRowsPerIter = (NT / kWave) * G * U;
    if (rows_per_wg <= 0) {
        // About two workgroups per CU on a 256-CU MI355X, in whole workgroup steps.
        const int want = (N + 511) / 512;
        rows_per_wg = std::max(kRowsPerIter, (want + kRowsPerIter - 1) / kRowsPerIter * kRowsPerIter);
    }
    const int nb = K >> 5;
    const size_t lds = static_cast<size_t>(M) * (K + 8 * nb);
    const int grid = (N + rows_per_wg - 1) / rows_per_wg;
    if (const hipError_t e = allow_lds(gemv_pairs_kernel<BB, LPR, U, MT, NT>, lds); e != hipSuccess) return e;
    hipLaunchKernelGGL((gemv_pairs_kernel<BB, LPR, U, MT, NT>), dim3(grid), dim3(NT), lds, stream, M, N, K, x, ldx, W,
                       y, ldy, rows_per_wg, acc);
    return hipGetLastError();
}

template <int BB, int U, int MT, int NT>
hipError_t launch_pairs_lpr(int lpr, int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y,
                            int ldy, int rows_per_wg, int acc, hipStream_t stream) {
    switch (lpr) {
        case 64: return launch_pairs<BB, 64, U, MT, NT>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, stream);
        case 32: return launch_pairs<BB, 32, U, MT, NT>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, stream);
        case 16: return launch_pairs<BB, 16, U, MT, NT>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, stream);
        default: return launch_pairs<BB, 8, U, MT, NT>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, stream);
    }
}

// One row of x: workgroup size and unroll are tunable.
template <int BB>
hipError_t launch_pairs_m1(int lpr, int nt, int u, int N, int K, const float* x, int ldx, const uint8_t* W, float* y,
                           int ldy, int rpw, int acc, hipStream_t s) {
#define SMK_PAIRS_M1(NT_, U_) \
    if (nt == NT_ && u == U_) return launch_pairs_lpr<BB, U_, 1, NT_>(lpr, 1, N, K, x, ldx, W, y, ldy, rpw, acc, s);
    SMK_PAIRS_M1(256, 1) SMK_PAIRS_M1(256, 2) SMK_PAIRS_M1(256, 4)
    SMK_PAIRS_M1(512, 1) SMK_PAIRS_M1(512, 2) SMK_PAIRS_M1(512, 4)
    SMK_PAIRS_M1(1024, 1) SMK_PAIRS_M1(1024, 2)
    // Four Q8_0 rows a lane group at 1024 threads would spill (68-byte pairs, 128 registers a lane).
    if constexpr (BB == kQ4_0Bytes) { SMK_PAIRS_M1(1024, 4) }
#undef SMK_PAIRS_M1
    return hipErrorInvalidValue;
}

template <int BB, int MT>
hipError_t launch_generic(int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y, int ldy,
                          int acc, hipStream_t stream) {
    const int rows_per_wg = 16;
    const int nb = K >> 5;
    const size_t lds = static_cast<size_t>(M) * (K + 8 * nb);
    const int grid = (N + rows_per_wg - 1) / rows_per_wg;
    if (const hipError_t e = allow_lds(gemv_generic_kernel<BB, MT>, lds); e != hipSuccess) return e;
    hipLaunchKernelGGL((gemv_generic_kernel<BB, MT>), dim3(grid), dim3(kThreads), lds, stream, M, N, K, x, ldx, W, y,
                       ldy, rows_per_wg, acc);
    return hipGetLastError();
}

// ─── Q4_0 launchers (the reference's SIMD order) ─────────────────────────────

inline bool accumulate_unsupported(int acc) { return acc != 0; }  // the SiLU-pair epilogue overwrites

size_t ordered_lds_bytes(int M, int K, int rows_per_group, int nbuf = 1) {
    const size_t nb = static_cast<size_t>(K) >> 5, quads = static_cast<size_t>(K) >> 2;
    const size_t x_words = ((M * (quads + nb) + 3) & ~static_cast<size_t>(3)) + M * nb * 4;
    return 4 * x_words + static_cast<size_t>(nbuf) * M * rows_per_group * ordered_stride(static_cast<int>(nb)) * 20;
}

struct NormArgs {
    const float* w = nullptr;
    double eps = 0.0;
    int depth = -1;
    int silu_pairs = 0;  // epilogue: rows (2n, 2n+1) -> y[n] = silu(row 2n) * row 2n+1
    int stream = 0;      // GemvTuning::stream_weights
};

template <int LPR, int MT, int NT, int CH, int kStream, bool kNorm>
hipError_t launch_ordered_kernel(int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y, int ldy,
                                 int rows_per_wg, int acc, const NormArgs& nrm, int nbuf, size_t lds,
                                 hipStream_t stream) {
    const int grid = (N + rows_per_wg - 1) / rows_per_wg;
    if (const hipError_t e = allow_lds(gemv_q4_ordered_kernel<LPR, MT, NT, CH, kStream, kNorm>, lds); e != hipSuccess)
        return e;
    hipLaunchKernelGGL((gemv_q4_ordered_kernel<LPR, MT, NT, CH, kStream, kNorm>), dim3(grid), dim3(NT), lds, stream, M, N,
                       K, x, ldx, W, y, ldy, rows_per_wg, acc, nrm.w, nrm.eps, nrm.depth, nrm.silu_pairs, nbuf);
    return hipGetLastError();
}

// Streamed weight groups (kStream of gemv_q4_ordered_kernel): SMK_Q4_STREAM=0 pair loads,
// 1 one group ahead, 2 two groups ahead (diagnostics, also set_q4_stream); unset: the built-in
// choice (-1).
std::atomic<int> g_q4_stream{[] {
    const char* v = std::getenv("SMK_Q4_STREAM");
    return v && v[0] >= '0' && v[0] <= '2' ? v[0] - '0' : -1;
}()};

template <int LPR, int MT, int NT, int CH>
hipError_t launch_ordered_ch(int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y, int ldy,
                             int rows_per_wg, int acc, const NormArgs& nrm, hipStream_t stream) {
    constexpr int kRows = NT / LPR;
    if (nrm.w && (M != 1 || (8 << nrm.depth) > NT)) return hipErrorInvalidValue;
    if (nrm.silu_pairs && (LPR > 32 || (rows_per_wg & 1) || accumulate_unsupported(acc))) return hipErrorInvalidValue;
    if (rows_per_wg <= 0) rows_per_wg = std::max(kRows, (N + 511) / 512);
    const size_t extra = nrm.w ? (static_cast<size_t>(K) + (8u << nrm.depth)) * 4 : 0;
    const size_t nb = static_cast<size_t>(K) >> 5;
    // Streamed groups: every row is whole 16-byte chunks (K % 256 == 0) and W is 16-byte
    // aligned, so a chunk that holds any byte of a workgroup's rows lies inside them; the
    // staging regions take kRows rows of LDS.
    const bool stream_shape = MT == 1 && CH <= 2 && g_q4_stream != 0 && nb % 8 == 0 &&
                              reinterpret_cast<uintptr_t>(W) % 16 == 0;
    const size_t stage = stream_shape ? kRows * nb * kQ4_0Bytes : 0;
    constexpr size_t kCap = 150 * 1024;
    // Two phase-1 buffers (phase 2 of a group overlaps the next group's phase 1) when a
    // workgroup has several groups and they fit.
    const int nbuf = (rows_per_wg > kRows && ordered_lds_bytes(M, K, kRows, 2) + extra + stage <= kCap) ? 2 : 1;
    const size_t lds = ordered_lds_bytes(M, K, kRows, nbuf) + extra;
    if constexpr (MT == 1 && CH <= 2) {
        const bool st = stream_shape && lds + stage <= kCap;
        const size_t bytes = lds + (st ? stage : 0);
        // Measured on MI355X (us, cached pair loads / one group ahead / two ahead): workgroups of
        // many groups stream best two ahead (lm_head 128256x2048 34.1 / 34.6 / 31.9); with a few
        // groups or one the cached pair loads are as fast or faster on their own (14336x4096
        // 11.1 / 11.5 / 11.8, 8192x2048 4.31 / 4.46 / 4.46), but inside a decode step one group
        // ahead is faster (1,557 / 1,616 tok/s with every GEMV in one mode): the non-temporal
        // weights leave the activations and the KV cache in the caches.
        const int groups = (rows_per_wg + kRows - 1) / kRows;
        const int forced = g_q4_stream.load();
        const int mode0 = !st ? 0 : forced > 0 ? forced : groups >= 8 ? 2 : nrm.stream ? 1 : 0;
        const int mode = NT == 1024 && mode0 == 2 ? 1 : mode0;  // (two groups ahead spill at 1024 threads)
#define SMK_ORDERED(S, NORM) \
    launch_ordered_kernel<LPR, MT, NT, CH, S, NORM>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, nrm, nbuf, bytes, stream)
        if constexpr (NT < 1024) {
            if (mode == 2) return nrm.w ? SMK_ORDERED(2, true) : SMK_ORDERED(2, false);
        }
        if (nrm.w) return mode == 1 ? SMK_ORDERED(1, true) : SMK_ORDERED(0, true);
        if (mode == 1) return SMK_ORDERED(1, false);
#undef SMK_ORDERED
    } else {
        if (nrm.w) return hipErrorInvalidValue;  // the fused norm covers K <= 8192: at most two pairs a lane
    }
    return launch_ordered_kernel<LPR, MT, NT, CH, 0, false>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, nrm, nbuf,
                                                            lds, stream);
}

// Pairs per lane and row: 1, 2, 4 or 8 (the lane split is raised until that suffices).
template <int LPR, int MT, int NT>
hipError_t launch_ordered(int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y, int ldy,
                          int rows_per_wg, int acc, hipStream_t stream, const NormArgs& nrm = NormArgs()) {
    const int chunks = ((K >> 6) + LPR - 1) / LPR;
    if constexpr (NT == 1024) {
        // 128 registers a lane: only one pair a lane and row, at least 16 lanes a row, and at
        // most one group in flight fit without spilling (the build checks it).
        if constexpr (LPR < 16) {
            return hipErrorInvalidValue;
        } else {
            if (chunks <= 1)
                return launch_ordered_ch<LPR, MT, NT, 1>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, nrm, stream);
            return hipErrorInvalidValue;
        }
    } else {
        if (chunks <= 1) return launch_ordered_ch<LPR, MT, NT, 1>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, nrm, stream);
        if (chunks <= 2) return launch_ordered_ch<LPR, MT, NT, 2>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, nrm, stream);
        if (chunks <= 4) return launch_ordered_ch<LPR, MT, NT, 4>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, nrm, stream);
        return hipErrorInvalidValue;
    }
}

template <int MT, int NT>
hipError_t launch_ordered_lpr(int lpr, int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y,
                              int ldy, int rows_per_wg, int acc, hipStream_t s, const NormArgs& nrm = NormArgs()) {
    switch (lpr) {
        case 64: return launch_ordered<64, MT, NT>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, s, nrm);
        case 32: return launch_ordered<32, MT, NT>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, s, nrm);
        case 16: return launch_ordered<16, MT, NT>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, s, nrm);
        default: return launch_ordered<8, MT, NT>(M, N, K, x, ldx, W, y, ldy, rows_per_wg, acc, s, nrm);
    }
}

// The tiled kernel (gemv_q4_tiled_kernel): 0 the built-in choice, -1 never, 2..4 that many
// tiles in flight wherever the shape allows it (diagnostics).
std::atomic<int> g_q4_tiles{0};

size_t tiled_lds_bytes(int K, int rows_per_wg, int acc) {
    return 4 * static_cast<size_t>(tiled_x_words(K)) + 2 * tiled::kPieces * 16 + 2 * tiled::kDotFloats * 4 +
           (acc ? 4 * static_cast<size_t>(rows_per_wg) : 0);
}

// One row of x, N even, K/32 a multiple of 8 (rows of whole 16-byte pieces), W 16-byte aligned,
// no fused norm, and the LDS image within 150 KiB (K up to about 37k).
bool tiled_ok(int K, const uint8_t* W, int rows_per_wg, int acc) {
    return g_q4_tiles >= 0 && (K >> 5) % 8 == 0 && reinterpret_cast<uintptr_t>(W) % 16 == 0 &&
           tiled_lds_bytes(K, rows_per_wg, acc) <= 150 * 1024;
}

template <int TF, int PQ, int XR, bool kNorm = false>
hipError_t launch_tiled_kernel(int N, int K, const float* x, const uint8_t* W, float* y, int rpw, int acc, int silu,
                               hipStream_t stream, const float* norm_w = nullptr, double norm_eps = 0.0) {
    const size_t lds = tiled_lds_bytes(K, rpw, acc);
    if (const hipError_t e = allow_lds(gemv_q4_tiled_kernel<TF, PQ, XR, kNorm>, lds); e != hipSuccess) return e;
    const int grid = (N + rpw - 1) / rpw;
    hipLaunchKernelGGL((gemv_q4_tiled_kernel<TF, PQ, XR, kNorm>), dim3(grid), dim3(tiled::kThreads), lds, stream, N, K,
                       x, W, y, rpw, acc, silu, norm_w, norm_eps);
    return hipGetLastError();
}

// x data in registers for rows of one or two chunks (K <= 4096), read from LDS otherwise.
template <int TF>
hipError_t launch_tiled_tf(int N, int K, const float* x, const uint8_t* W, float* y, int rpw, int acc, int silu,
                           hipStream_t stream) {
    const int chunks = ((K >> 5) + tiled::kBlocks - 1) / tiled::kBlocks;
    const int pq = ((K >> 3) + tiled::kThreads - 1) / tiled::kThreads;  // octs of x per thread
    if (chunks == 1) return launch_tiled_kernel<TF, 1, 1>(N, K, x, W, y, rpw, acc, silu, stream);
    if constexpr (TF == 2)  // (two chunks in registers and four tiles in flight would spill)
        if (chunks == 2) return launch_tiled_kernel<TF, 1, 2>(N, K, x, W, y, rpw, acc, silu, stream);
    if (pq <= 1) return launch_tiled_kernel<TF, 1, 0>(N, K, x, W, y, rpw, acc, silu, stream);
    if (pq <= 2) return launch_tiled_kernel<TF, 2, 0>(N, K, x, W, y, rpw, acc, silu, stream);
    return launch_tiled_kernel<TF, 4, 0>(N, K, x, W, y, rpw, acc, silu, stream);  // octs past 4 a thread: loop
}

hipError_t launch_tiled(int N, int K, const float* x, const uint8_t* W, float* y, int rpw, int acc, int silu,
                        hipStream_t stream) {
    const int forced = g_q4_tiles.load();
    const int tf = forced >= 2 ? forced : 2;
    switch (tf) {
        case 3: return launch_tiled_tf<3>(N, K, x, W, y, rpw, acc, silu, stream);
        case 4: return launch_tiled_tf<4>(N, K, x, W, y, rpw, acc, silu, stream);
        default: return launch_tiled_tf<2>(N, K, x, W, y, rpw, acc, silu, stream);
    }
}

template <int MT>
hipError_t launch_ordered_generic(int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y, int ldy,
                                  int acc, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(M) * ((K >> 2) + (K >> 5)) * 4;
    const int grid = (N + kThreads / 4 - 1) / (kThreads / 4);
    if (const hipError_t e = allow_lds(gemv_q4_ordered_generic_kernel<MT>, lds); e != hipSuccess) return e;
    hipLaunchKernelGGL(gemv_q4_ordered_generic_kernel<MT>, dim3(grid), dim3(kThreads), lds, stream, M, N, K, x, ldx,
                       W, y, ldy, acc);
    return hipGetLastError();
}

hipError_t gemv_q4_ordered(int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y, int ldy,
                           hipStream_t stream, const GemvTuning* t) {
    const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
    const int acc = t ? t->accumulate : 0;
    const int pairs = (K >> 5) / 2;
    constexpr size_t kLdsCap = 150 * 1024;
    // Rows of more than 4 * 64 pairs (K > 16384) that the tiled kernel does not take go to the
    // generic kernel: eight pairs a lane would not fit the row-group kernel's registers.
    const bool generic = !pair_path_ok(K, W) || ordered_lds_bytes(M, K, 256 / 64) > kLdsCap || pairs > 4 * 64;
    NormArgs nrm;
    nrm.stream = t ? t->stream_weights : 0;
    if (t && t->silu_pairs) {
        if (M != 1 || generic || (N & 1)) return hipErrorInvalidValue;
        nrm.silu_pairs = 1;
    }
    if (t && t->norm_w) {
        // Fused RMSNorm: one row of x, K <= 8192, the pair kernel (even N), a uniform tree of
        // equal leaves.
        nrm.w = t->norm_w;
        nrm.eps = t->norm_eps;
        nrm.depth = uniform_depth(K);
        if (M != 1 || K > 8192 || !uniform_equal_leaves(K, nrm.depth) || generic || (N & 1) ||
            (8 << nrm.depth) > 1024 ||
            reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(t->norm_w) % 16)
            return hipErrorInvalidValue;
    }
    if (!generic && (N & 1)) {
        // The last row of an odd N has its own order (q4_row_single): one row through the
        // generic kernel, the even rest through the pair kernel.
        const size_t row_bytes = static_cast<size_t>(K >> 5) * kQ4_0Bytes;
        hipError_t e = hipSuccess;
        switch (mt) {
            case 1: e = launch_ordered_generic<1>(M, 1, K, x, ldx, W + (N - 1) * row_bytes, y + (N - 1), ldy, acc, stream); break;
            case 2: e = launch_ordered_generic<2>(M, 1, K, x, ldx, W + (N - 1) * row_bytes, y + (N - 1), ldy, acc, stream); break;
            case 4: e = launch_ordered_generic<4>(M, 1, K, x, ldx, W + (N - 1) * row_bytes, y + (N - 1), ldy, acc, stream); break;
            default: e = launch_ordered_generic<8>(M, 1, K, x, ldx, W + (N - 1) * row_bytes, y + (N - 1), ldy, acc, stream); break;
        }
        if (e != hipSuccess || N == 1) return e;
        --N;
    }
    if (generic) {
        switch (mt) {
            case 1: return launch_ordered_generic<1>(M, N, K, x, ldx, W, y, ldy, acc, stream);
            case 2: return launch_ordered_generic<2>(M, N, K, x, ldx, W, y, ldy, acc, stream);
            case 4: return launch_ordered_generic<4>(M, N, K, x, ldx, W, y, ldy, acc, stream);
            default: return launch_ordered_generic<8>(M, N, K, x, ldx, W, y, ldy, acc, stream);
        }
    }
    // The lane split does not change the result here (every row's sum has the reference's
    // order), so it is chosen for speed only.
    // Measured on MI355X: one workgroup per compute unit (its groups pipelined through two
    // phase-1 buffers), 32 lanes per row up to 32 pairs a row and 64 beyond, and the fewest
    // threads (256 or 512) whose group covers the workgroup's rows, else 512 (1024 threads, 128
    // registers a lane, spilled in most forms and measured no faster: decode 1,697 tok/s either way,
    // lm_head 128256x2048 30.8 / 30.7 us).
    int lpr = (t && t->lanes_per_row) ? t->lanes_per_row : (pairs >= 64 ? 64 : pairs >= 16 ? 32 : 16);
    while (lpr < 64 && (pairs + lpr - 1) / lpr > 4) lpr *= 2;  // at most 4 pairs per lane and row
    int rpw = t ? t->rows_per_wg : 0;
    if (rpw <= 0) {
        rpw = std::max(1, (N + g_cus - 1) / g_cus);
        rpw += rpw & 1;  // (gate, up) pairs of the SiLU epilogue never straddle workgroups
    }
    // The K-chunk tiled kernel where it measured faster on MI355X (graph-replayed, us, tiled /
    // row-group): long rows, 4096x14336 12.1 / 16.0; many rows a workgroup, 128256x4096 56.0 / 58.8.
    // Short rows and few rows keep the row-group kernel (8192x2048 5.68 / 4.12, 16384x2048 7.55 /
    // 5.67, 3072x2048 3.98 / 3.35, 2048x2048 3.94 / 3.22, 2048x8192 7.40 / 5.53, 14336x4096 11.0 /
    // 10.4): its one or two groups need fewer barriers.
    const bool tiled_pays = g_q4_tiles > 0 || K >= 12288 || rpw >= 256;
    // The fused norm in the tiled kernel: K = 2048 (one chunk, the one-wave mean of squares).
    const bool tiled_norm = nrm.w && K == 2048 && nrm.depth == 4 && !acc && !nrm.silu_pairs;
    if (mt == 1 && (!nrm.w || tiled_norm) && !(t && (t->lanes_per_row || t->threads)) && tiled_pays &&
        tiled_ok(K, W, rpw, acc) && !(nrm.silu_pairs && (rpw & 1))) {
        if (nrm.w) return launch_tiled_kernel<2, 1, 1, true>(N, K, x, W, y, rpw, 0, 0, stream, nrm.w, nrm.eps);
        return launch_tiled(N, K, x, W, y, rpw, acc, nrm.silu_pairs, stream);
    }
    if (mt == 1) {
        if (nrm.silu_pairs) {
            if (rpw & 1) return hipErrorInvalidValue;
            if (lpr > 32) lpr = 32;    // two rows at least side by side in a wave
        }
        int nt = (t && t->threads) ? t->threads : 256;
        const size_t cap = kLdsCap - (nrm.w ? (static_cast<size_t>(K) + (8u << nrm.depth)) * 4 : 0);
        if (!(t && t->threads)) {
            while (nt < 1024 && nt < rpw * lpr) nt *= 2;
            if (nt == 1024 && (lpr < 16 || pairs > lpr)) nt = 512;  // the 1024-thread forms that fit
            while (nt > 256 && ordered_lds_bytes(1, K, nt / lpr) > cap) nt /= 2;
        }
        while (ordered_lds_bytes(1, K, nt / lpr) > cap && lpr < (nrm.silu_pairs ? 32 : 64)) lpr *= 2;
        if (nrm.w)  // eight lanes per leaf of the norm's tree, at most four quads of x per thread
            while (nt < (8 << nrm.depth) || nt * 16 < K) nt *= 2;
        switch (nt) {
            case 1024: return launch_ordered_lpr<1, 1024>(lpr, M, N, K, x, ldx, W, y, ldy, rpw, acc, stream, nrm);
            case 512: return launch_ordered_lpr<1, 512>(lpr, M, N, K, x, ldx, W, y, ldy, rpw, acc, stream, nrm);
            case 256: return launch_ordered_lpr<1, 256>(lpr, M, N, K, x, ldx, W, y, ldy, rpw, acc, stream, nrm);
            default: return hipErrorInvalidValue;
        }
    }
    // Several rows of x: 256 threads, 32 or 64 lanes per row (phase 2 needs 4 * rows * M <= 256).
    const bool l32 = ordered_lds_bytes(M, K, 256 / 32) <= kLdsCap && (!(t && t->lanes_per_row) || lpr <= 32);
    switch (mt) {
        case 2: return l32 ? launch_ordered<32, 2, 256>(M, N, K, x, ldx, W, y, ldy, rpw, acc, stream)
                           : launch_ordered<64, 2, 256>(M, N, K, x, ldx, W, y, ldy, rpw, acc, stream);
        case 4: return l32 ? launch_ordered<32, 4, 256>(M, N, K, x, ldx, W, y, ldy, rpw, acc, stream)
                           : launch_ordered<64, 4, 256>(M, N, K, x, ldx, W, y, ldy, rpw, acc, stream);
        default: return l32 ? launch_ordered<32, 8, 256>(M, N, K, x, ldx, W, y, ldy, rpw, acc, stream)
                            : launch_ordered<64, 8, 256>(M, N, K, x, ldx, W, y, ldy, rpw, acc, stream);
    }
}

template <int BB>
hipError_t gemv_quant_fmt(int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y, int ldy,
                          hipStream_t stream, const GemvTuning* t) {
    if constexpr (BB == kQ4_0Bytes) {
        if (!(t && t->unordered)) return gemv_q4_ordered(M, N, K, x, ldx, W, y, ldy, stream, t);
    }
    const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
    const int acc = t ? t->accumulate : 0;
    if (!pair_path_ok(K, W)) {
        switch (mt) {
            case 1: return launch_generic<BB, 1>(M, N, K, x, ldx, W, y, ldy, acc, stream);
            case 2: return launch_generic<BB, 2>(M, N, K, x, ldx, W, y, ldy, acc, stream);
            case 4: return launch_generic<BB, 4>(M, N, K, x, ldx, W, y, ldy, acc, stream);
            default: return launch_generic<BB, 8>(M, N, K, x, ldx, W, y, ldy, acc, stream);
        }
    }
    // The lane split fixes the summation order, so it depends on the shape only: every row of a
    // batched call then equals the single-row call bit for bit.  64 lanes per row once a row
    // holds >= 128 pairs, or >= 64 pairs with N <= 4096; else 32 (measured best on MI355X for the
    // BASELINE and Llama-3-8B shapes: Q8_0 4096x4096 5.68 -> 5.20 us with 64).
    const int pairs = (K >> 5) / 2;
    const int lpr = (t && t->lanes_per_row)
                        ? t->lanes_per_row
                        : (pairs >= 128 || (pairs >= 64 && N <= 4096) ? 64 : (pairs >= 32 ? 32 : choose_lpr(pairs)));
    int rpw = t ? t->rows_per_wg : 0;
    if (mt == 1) {
        // One row of x (decode).  Measured on MI355X over the BASELINE shapes (9.4 MB to 295 MB
        // of weights): one pair per lane per step; 1024-thread workgroups for small and very
        // large matrices, 512 in between; 1, 2 or 4 workgroups per CU with the rows split evenly.
        // Rows of K >= 8192: one workgroup per CU (Q8_0 4096x14336 15.1 -> 13.9 us).
        const double bytes = static_cast<double>(N) * (K >> 5) * BB;
        const bool one = bytes < 24e6 || K >= 8192;
        const int nt_auto = (one || bytes >= 128e6) ? 1024 : 512;
        const int per_cu = one ? 1 : (bytes < 128e6 ? 2 : 4);
        if (rpw <= 0) rpw = std::max(1, (N + g_cus * per_cu - 1) / (g_cus * per_cu));
        // No more waves than rows: a wave covers 64 / lpr rows per step.
        int nt = (t && t->threads) ? t->threads : nt_auto;
        if (!(t && t->threads))
            while (nt > 256 && nt > rpw * lpr) nt /= 2;
        const int u = (t && t->unroll) ? t->unroll : 1;
        return launch_pairs_m1<BB>(lpr, nt, u, N, K, x, ldx, W, y, ldy, rpw, acc, stream);
    }
    constexpr int U2 = BB == kQ4_0Bytes ? 4 : 2, U4 = BB == kQ4_0Bytes ? 2 : 1;
    switch (mt) {
        case 2: return launch_pairs_lpr<BB, U2, 2, 256>(lpr, M, N, K, x, ldx, W, y, ldy, rpw, acc, stream);
        case 4: return launch_pairs_lpr<BB, U4, 4, 256>(lpr, M, N, K, x, ldx, W, y, ldy, rpw, acc, stream);
        default: return launch_pairs_lpr<BB, U4, 8, 256>(lpr, M, N, K, x, ldx, W, y, ldy, rpw, acc, stream);
    }
}

}  // namespace

hipError_t fill(float* y, long long n, float value, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int grid = static_cast<int>(std::min<long long>((n + 255) / 256, 1024));
    hipLaunchKernelGGL(fill_kernel, dim3(grid), dim3(256), 0, stream, y, n, value);
    return hipGetLastError();
}

hipError_t gemv_quant(int block_bytes, int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y,
                      int ldy, hipStream_t stream, const GemvTuning* tuning) {
    if (N <= 0 || M <= 0) return hipSuccess;
    if (K < 0 || K % 32 != 0) return hipErrorInvalidValue;
    if (K == 0) {
        if (tuning && tuning->accumulate) return hipSuccess;  // y + 0
        for (int m = 0; m < M; ++m) {
            const hipError_t e = fill(y + static_cast<size_t>(m) * ldy, N, 0.0f, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    if (block_bytes != kQ4_0Bytes && block_bytes != kQ8_0Bytes) return hipErrorInvalidValue;
    if (block_bytes == kQ4_0Bytes && M > 1 && !(tuning && (tuning->unordered || tuning->norm_w || tuning->silu_pairs)) &&
        (tuning && tuning->mfma_min_rows ? M >= tuning->mfma_min_rows : (M >= kMfmaMinRows && mfma_rows_pay(M, N)))) {
        // Several rows of x on the matrix cores; the last row of an odd N (its own order) goes
        // through the one-row kernels below.
        const int ne = N & ~1;
        if (ne > 0 && gemm_q4_mfma_ok(M, ne, K, W)) {
            void* ws = nullptr;
            if (tuning && tuning->workspace) {  // the caller's scratch: never allocate
                if (gemm_q4_mfma_workspace(M, K) > tuning->workspace_bytes) return hipErrorInvalidValue;
                ws = tuning->workspace;
            } else if (const hipError_t e = stream_workspace(stream, gemm_q4_mfma_workspace(M, K), &ws);
                       e != hipSuccess) {
                return e;
            }
            const hipError_t e = gemm_q4_mfma(M, ne, K, x, ldx, W, y, ldy, tuning ? tuning->accumulate : 0, ws, stream);
            if (e != hipSuccess || ne == N) return e;
            const size_t row_bytes = static_cast<size_t>(K >> 5) * kQ4_0Bytes;
            return gemv_quant(block_bytes, M, 1, K, x, ldx, W + ne * row_bytes, y + ne, ldy, stream, tuning);
        }
    }
    // The x quants of one launch live in LDS (K + 8*K/32 bytes per row of x): split the rows of
    // x so that each launch fits in 144 KiB of the CU's 160 KiB.
    const size_t per_row = static_cast<size_t>(K) + 8 * static_cast<size_t>(K >> 5);
    const int rows_fit = static_cast<int>(std::min<size_t>(8, (144 * 1024) / per_row));
    if (rows_fit < 1) return hipErrorInvalidValue;  // K > ~117k
    for (int m0 = 0; m0 < M; m0 += rows_fit) {
        const int mr = std::min(rows_fit, M - m0);
        const float* xm = x + static_cast<size_t>(m0) * ldx;
        float* ym = y + static_cast<size_t>(m0) * ldy;
        const hipError_t e = block_bytes == kQ4_0Bytes
                                 ? gemv_quant_fmt<kQ4_0Bytes>(mr, N, K, xm, ldx, W, ym, ldy, stream, tuning)
                                 : gemv_quant_fmt<kQ8_0Bytes>(mr, N, K, xm, ldx, W, ym, ldy, stream, tuning);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

const char* gemv_quant_path(int, int, int K, const uint8_t* W) { return pair_path_ok(K, W) ? "pairs" : "generic"; }

void set_compute_units(int cus) { g_cus = cus > 0 ? cus : 256; }

void set_q4_stream(int mode) { g_q4_stream = mode; }

void set_q4_tiles(int tiles) { g_q4_tiles = tiles; }

hipError_t quantize_x_q8(int K, const float* x, int8_t* qs, float* dx, int* bad, hipStream_t stream) {
    if (K <= 0) return hipSuccess;
    const int nb = K >> 5;
    const int grid = (nb + 31) / 32;
    hipLaunchKernelGGL(quantize_x_kernel, dim3(grid), dim3(kThreads), 32 * 32 + 8 * 32, stream, K, x, qs, dx, bad);
    return hipGetLastError();
}

hipError_t block_sums(int block_bytes, int N, int K, const int8_t* qs, const uint8_t* W, int32_t* out,
                      hipStream_t stream) {
    const long long total = static_cast<long long>(N) * (K >> 5);
    if (total <= 0) return hipSuccess;
    const int grid = static_cast<int>(std::min<long long>((total + 255) / 256, 4096));
    if (block_bytes == kQ4_0Bytes)
        hipLaunchKernelGGL(block_sums_kernel<kQ4_0Bytes>, dim3(grid), dim3(256), 0, stream, N, K, qs, W, out);
    else
        hipLaunchKernelGGL(block_sums_kernel<kQ8_0Bytes>, dim3(grid), dim3(256), 0, stream, N, K, qs, W, out);
    return hipGetLastError();
}

}  // namespace smk
