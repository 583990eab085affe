// decoder.hip -- device-resident Llama decode step for gfx950: the per-token loop of
// examples/llama/llama.py (step :414-439, _attention :398-412, generate :481-505) with every
// weight, activation and the KV cache in HBM, and one HIP graph per token.
//
// Per layer, the step runs (llama.py:428-434):
//   h = rms_norm(x, attn_norm)                   in the GEMV's prologue (numpy-exact; Q4_0),
//   [q|k|v] = h @ [Wq;Wk;Wv]^T                   one GEMV over the three matrices' rows
//   q, k = rope(q), rope(k); cache[pos] = k, v   in attention_kernel
//   a = attention(q, cache[0..pos])              attention_kernel (one workgroup per head)
//   x = x + a @ Wo^T                             GEMV with a residual epilogue
//   h = rms_norm(x, mlp_norm)                    in the GEMV's prologue
//   [g|u] = h @ [Wgate;Wup]^T                    one GEMV
//   x = x + (silu(g) * u) @ Wdown^T              silu_mul_kernel, GEMV with residual epilogue
// then logits = rms_norm(x, norm) @ lm_head^T and the greedy argmax on the device.
//
// Rows of a GEMV are independent and the lane split depends on K only, so the fused
// [q|k|v] and [g|u] products equal the separate per-matrix calls bit for bit.  The position
// and the token of a step live in device memory (DecodeState, the token array): a captured
// graph replays unchanged for every position, and generate() runs prompt and decode steps
// back to back with no host round trip.
#include "abi_internal.hpp"
#include "device_common.hpp"
#include "launch.hpp"
#include "pairwise_sum.hpp"
#include "smk_hip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

namespace smk {
namespace {

constexpr int kGgmlF32 = 0, kGgmlQ4_0 = 2, kGgmlQ8_0 = 8;
constexpr int kMaxCapacity = 16384;  // attention scores of one head live in LDS

struct DecodeState {
    int pos;       // position of the next step
    int n_prompt;  // tokens[0, n_prompt) are given; argmax fills the rest
};

// ─── kernels ────────────────────────────────────────────────────────────────

// x = row `token` of the embedding (llama.py:337 / gguf_reader.py:112-129: d * (q - 8) for
// Q4_0, d * q for Q8_0, the float32 row for F32; every product is exact in float32).  One thread
// per 32-value block: all 2-byte reads of the block are issued before any value is formed (GGUF
// blocks are 2-byte aligned), so a row costs one memory latency, not one per value.
__device__ __forceinline__ void embed_row(const uint8_t* __restrict__ E, int type, int hidden, int vocab, int tok,
                                          float* __restrict__ x) {
    tok = min(max(tok, 0), vocab - 1);  // host checks every token; a bad one must not fault
    if (type == kGgmlF32) {  // any width
        const float* src = reinterpret_cast<const float*>(E) + static_cast<size_t>(tok) * hidden;
        for (int i = threadIdx.x; i < hidden; i += blockDim.x) x[i] = src[i];
        return;
    }
    const int nb = hidden >> 5;  // quantized rows are whole blocks
    for (int b = threadIdx.x; b < nb; b += blockDim.x) {
        float v[32];
        if (type == kGgmlQ4_0) {
            const uint16_t* blk = reinterpret_cast<const uint16_t*>(E + (static_cast<size_t>(tok) * nb + b) * kQ4_0Bytes);
            uint16_t h[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) h[k] = blk[k];
            const float d = half_bits_to_float(h[0]);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int byte = (h[1 + (j >> 1)] >> (8 * (j & 1))) & 0xff;
                v[j] = d * static_cast<float>((byte & 15) - 8);
                v[16 + j] = d * static_cast<float>((byte >> 4) - 8);
            }
        } else {
            const uint16_t* blk = reinterpret_cast<const uint16_t*>(E + (static_cast<size_t>(tok) * nb + b) * kQ8_0Bytes);
            uint16_t h[17];
#pragma unroll
            for (int k = 0; k < 17; ++k) h[k] = blk[k];
            const float d = half_bits_to_float(h[0]);
#pragma unroll
            for (int j = 0; j < 32; ++j)
                v[j] = d * static_cast<float>(static_cast<int8_t>((h[1 + (j >> 1)] >> (8 * (j & 1))) & 0xff));
        }
#pragma unroll
        for (int j = 0; j < 32; ++j) x[32 * b + j] = v[j];
    }
}

__global__ void embed_kernel(const uint8_t* __restrict__ E, int type, int hidden, int vocab,
                             const int* __restrict__ tokens, const DecodeState* __restrict__ st,
                             float* __restrict__ x) {
    embed_row(E, type, hidden, vocab, tokens[st->pos], x);
}

// Rows p < gridDim.x of a prompt chunk: x[p] = row tokens[p] of the embedding.
__global__ void embed_rows_kernel(const uint8_t* __restrict__ E, int type, int hidden, int vocab,
                                  const int* __restrict__ tokens, float* __restrict__ x) {
    embed_row(E, type, hidden, vocab, tokens[blockIdx.x], x + static_cast<size_t>(blockIdx.x) * hidden);
}

// Grouped-query attention of one query head over positions 0..pos (llama.py:398-412) with the
// RoPE of the step folded in, in the arithmetic order of the reference's SIMD tables, so that
// every score, probability and output equals the reference's bit for bit:
//   q, k = rope(q), rope(k) (llama.py:387-396 interleaved, :169-178 half split; numpy's
//     separate roundings); the first workgroup of each KV group writes k and v into the cache at
//     pos, and every workgroup uses its own copies for position pos (same values);
//   scores = sk.sgemm(q, K, alpha=scale, trans_b=True): the AVX-512 few-row dot
//     (avx512_gemm_packed.cpp:216-240): 16 lanes per dot, lane l accumulating products
//     p = l, l+32, ... and 16+l, 48+l, ... in two fused chains, the two chains added, the 16
//     sums reduced by halves (lanes i and i+8, i and i+4, i and i+2, then the pair), times scale;
//   p = sk.softmax(scores): softmax_row_avx2's order (the exp of simd_math.hpp on full groups
//     of 8, eight running double sums, a double exp on the last n % 8);
//   out = sk.sgemm(p, V): the AVX2 direct product (avx2_gemm_packed.cpp:151-201), one fused
//     chain over the positions in order per output.
// One workgroup of kAttnThreads threads per query head; scores in LDS; cached K and V read in tiles of
// `tile` positions staged through LDS (up to kMaxTile; every position of a decode that fits
// one tile is read in the first round, together with q, k and v).
constexpr int kAttnThreads = 512;  // measured: 256 / 512 / 1024 threads, decode 1,694 / 1,715 / 1,675 tok/s
constexpr int kHeadMax = 256;     // head_dim limit (create() checks it)
constexpr int kRopeKvThreads = 256;
constexpr int kMaxTile = 256;
constexpr size_t kAttnLdsBudget = 150 * 1024;

// Row stride (floats) of the K tile in LDS: one thread reads a whole row for its score, and at
// this stride the rows of 16 neighbouring lanes start in different banks.
__host__ __device__ __forceinline__ int k_stride(int hd) { return hd + 4; }

// count floats (a multiple of 4, 16-byte aligned ends) from global to LDS in batches of R rounds
// of kAttnThreads x 16 bytes (of each source): every thread issues a batch's loads before storing
// any. Every store is unconditional (an element past the end goes to the spare slot `dump`): a
// load whose only use is a store under a branch is moved by the compiler into that branch, and
// the rounds then wait for each other one at a time.  d0 takes rows of row4 float4s at a stride
// of d0_stride floats; d1 is dense.
template <bool kTwo, int R>  // kTwo: d1 from s1 as well
__device__ __forceinline__ void stage_rounds(float* __restrict__ d0, const float* __restrict__ s0,
                                             float* __restrict__ d1, const float* __restrict__ s1, int count,
                                             float* __restrict__ dump, int row4, int d0_stride) {
    const float4* a4 = reinterpret_cast<const float4*>(s0);
    const float4* b4 = reinterpret_cast<const float4*>(s1);
    const int n4 = count >> 2;
    for (int base = 0; base < n4; base += R * kAttnThreads) {
        float4 va[R], vb[R];
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const int e = base + u * kAttnThreads + static_cast<int>(threadIdx.x);
            va[u] = a4[e < n4 ? e : 0];
            if constexpr (kTwo) vb[u] = b4[e < n4 ? e : 0];
        }
#pragma unroll
        for (int u = 0; u < R; ++u) {
            const int e = base + u * kAttnThreads + static_cast<int>(threadIdx.x);
            const int r = e / row4;
            *reinterpret_cast<float4*>(e < n4 ? d0 + r * d0_stride + 4 * (e - r * row4) : dump) = va[u];
            if constexpr (kTwo) *reinterpret_cast<float4*>(e < n4 ? d1 + 4 * e : dump) = vb[u];
        }
    }
}
// Four rounds a batch, or eight when the data needs more than four (one wait for a whole tile of
// 256 positions of head_dim 64).
template <bool kTwo>
__device__ __forceinline__ void stage_tiles(float* __restrict__ d0, const float* __restrict__ s0,
                                            float* __restrict__ d1, const float* __restrict__ s1, int count,
                                            float* __restrict__ dump, int row4, int d0_stride) {
    if (count > 16 * kAttnThreads)
        stage_rounds<kTwo, 8>(d0, s0, d1, s1, count, dump, row4, d0_stride);
    else
        stage_rounds<kTwo, 4>(d0, s0, d1, s1, count, dump, row4, d0_stride);
}

// The score of one position, computed by one thread: the reference's 16-lane dot (element e
// goes to lane e % 16, chain (e / 16) % 2, each chain fused in increasing e from +0), the two
// chains of a lane added, the 16 lane sums reduced by halves (lanes i and i+8, i and i+4, i and
// i+2, then the pair), times scale.  q is read from LDS at the same address by every lane; kr is
// the position's row of the K tile.  HD > 0: head_dim HD; 0: hd at run time.
template <int HD>
__device__ __forceinline__ float position_score(const float* __restrict__ qs, const float* __restrict__ kr, int hd,
                                                float scale) {
    float a[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) a[i] = 0.0f;
    const float4* q4 = reinterpret_cast<const float4*>(qs);
    const float4* k4 = reinterpret_cast<const float4*>(kr);
    // 32 elements a step (both chains of every lane once); within a step the chain of each
    // element is a constant.
    auto step = [&](int p, int n) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (p + 4 * j < n) {
                const float4 q = q4[p / 4 + j], k = k4[p / 4 + j];
                const float qv[4] = {q.x, q.y, q.z, q.w}, kv[4] = {k.x, k.y, k.z, k.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int e = 4 * j + i;  // element p + e: lane e % 16, chain e / 16
                    a[(e >> 4) * 16 + (e & 15)] = fmaf(qv[i], kv[i], a[(e >> 4) * 16 + (e & 15)]);
                }
            }
        }
    };
    if constexpr (HD > 0) {
#pragma unroll
        for (int p = 0; p < HD; p += 32) step(p, HD);
    } else {
        for (int p = 0; p < hd; p += 32) step(p, hd);
    }
    float v[16];
#pragma unroll
    for (int l = 0; l < 16; ++l) v[l] = a[l] + a[16 + l];
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1) {
#pragma unroll
        for (int l = 0; l < w; ++l) v[l] = v[l] + v[l + w];
    }
    return scale * v[0];
}

// v of lane l as a wave-uniform value.
__device__ __forceinline__ double readlane_d(double v, int l) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
    const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(u & 0xffffffffu), l));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), l));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// 0.0 + f[0] + f[8] + ... + f[8 (n - 1)], in double, in order.  The reads in batches of eight in
// two register sets used in turn (each batch's reads issued before the previous batch's adds);
// the last n % 8 values, read with clamped indices, are issued first of all.
template <bool kClamp>
__device__ __forceinline__ void dsum_load(const float* __restrict__ f, int n, int i0, float (&r)[8]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) r[u] = f[8 * (kClamp ? min(i0 + u, n - 1) : i0 + u)];
}
__device__ __forceinline__ double dsum_add(const float (&r)[8], double acc, int live = 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u)
        if (u < live) acc = acc + static_cast<double>(r[u]);
    return acc;
}
__device__ __forceinline__ double strided_dsum(const float* __restrict__ f, int n) {
    double acc = 0.0;
    const int nb = n >> 3, rem = n & 7;
    if (n == 0) return acc;
    // Both issued unconditionally, with no branch between them (the first batch's reads stay
    // among the values that the caller's f holds).
    float tl[8], a[8], b[8];
    dsum_load<true>(f, n, 8 * nb, tl);
    dsum_load<true>(f, n, 0, a);
    __builtin_amdgcn_sched_barrier(0);
    if (nb > 0) {
        int k = 1;  // a holds batch k - 1
        for (; k + 1 < nb; k += 2) {
            dsum_load<false>(f, n, 8 * k, b);
            __builtin_amdgcn_sched_barrier(0);
            acc = dsum_add(a, acc);
            dsum_load<false>(f, n, 8 * k + 8, a);
            __builtin_amdgcn_sched_barrier(0);
            acc = dsum_add(b, acc);
        }
        if (k < nb) {
            dsum_load<false>(f, n, 8 * k, b);
            __builtin_amdgcn_sched_barrier(0);
            acc = dsum_add(a, acc);
            acc = dsum_add(b, acc);
        } else {
            acc = dsum_add(a, acc);
        }
    }
    return rem ? dsum_add(tl, acc, rem) : acc;
}

// Eight positions of the p.V chain from position t: p[t .. t + 7] (16-byte aligned; the reads may
// pass the n positions, into LDS that the kernel owns) and rows t .. t + 7 of v (kClamp: clamped
// to row n - 1).
struct PvBatch {
    float4 a, b;
    float w[8];
};
template <int HD, bool kClamp>
__device__ __forceinline__ void pv_load(const float* __restrict__ p, const float* __restrict__ v, int hd_arg, int n,
                                        int t, PvBatch& o) {
    const int hd = HD > 0 ? HD : hd_arg;
    const float4* p4 = reinterpret_cast<const float4*>(p + t);
    o.a = p4[0];
    o.b = p4[1];
#pragma unroll
    for (int i = 0; i < 8; ++i) o.w[i] = v[(kClamp ? min(t + i, n - 1) : t + i) * hd];
}
// The batch's first `live` positions (all eight by default) into the chain, in order.
__device__ __forceinline__ float pv_fma(const PvBatch& o, float acc, int live = 8) {
    const float pp[8] = {o.a.x, o.a.y, o.a.z, o.a.w, o.b.x, o.b.y, o.b.z, o.b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (i < live) acc = fmaf(pp[i], o.w[i], acc);
    return acc;
}

// acc after the fused chain acc = fma(p[t], v[t * hd], acc) for t = 0 .. n - 1 in order (p 16-byte
// aligned, readable to 8 floats past n rounded down to 8).  Eight positions a batch in two
// register sets used in turn: the reads of the next batch are issued before the FMAs of the
// current one and stay in flight across the loop, so that the chain waits on LDS once per batch
// at most, not once per position.  The last n % 8 positions are read first of all.
template <int HD>
__device__ __forceinline__ float pv_chain(const float* __restrict__ p, const float* __restrict__ v, int n, int hd_arg,
                                          float acc) {
    const int hd = HD > 0 ? HD : hd_arg;
    const int nb = n >> 3, rem = n & 7;
    // Both issued unconditionally, with no branch between them (n >= 1; with n < 8 the first
    // batch reads rows 0 .. 7 of a tile of at least 16 rows and is not used).
    PvBatch tl, s0, s1;
    pv_load<HD, true>(p, v, hd, n, 8 * nb, tl);
    pv_load<HD, false>(p, v, hd, n, 0, s0);
    __builtin_amdgcn_sched_barrier(0);
    if (nb > 0) {
        int b = 1;  // s0 holds batch b - 1
        for (; b + 1 < nb; b += 2) {
            pv_load<HD, false>(p, v, hd, n, 8 * b, s1);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv_fma(s0, acc);
            pv_load<HD, false>(p, v, hd, n, 8 * b + 8, s0);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv_fma(s1, acc);
        }
        if (b < nb) {
            pv_load<HD, false>(p, v, hd, n, 8 * b, s1);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv_fma(s0, acc);
            acc = pv_fma(s1, acc);
        } else {
            acc = pv_fma(s0, acc);
        }
    }
    return rem ? pv_fma(tl, acc, rem) : acc;
}

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(const float* __restrict__ qkv,
                                                                 const float* __restrict__ cos_tab,
                                                                 const float* __restrict__ sin_tab, int interleaved,
                                                                 float* __restrict__ kc, float* __restrict__ vc,
                                                                 int n_heads, int n_kv, int hd_arg, int cap,
                                                                 float scale, int tile,
                                                                 const DecodeState* __restrict__ st,
                                                                 float* __restrict__ out, int pos_first,
                                                                 int qkv_stride, int out_stride) {
    constexpr int kWaves = kAttnThreads / kWave;
    extern __shared__ __align__(16) float sc[];  // T scores, exponentials, then p; then the K and V tiles
    __shared__ __align__(16) float qs[kHeadMax];
    __shared__ float ks[kHeadMax], vs[kHeadMax];
    __shared__ float red_f[kWaves];
    __shared__ int red_i[kWaves];
    __shared__ double tail_e[8];
    __shared__ float inv_s;
    const int hd = HD > 0 ? HD : hd_arg, kst = k_stride(hd);
    // Workgroup b takes KV group b % n_kv: the workgroups of one group are n_kv apart, and with
    // workgroups dealt to the XCDs in turn (8 on MI355X) they share an XCD, and so its L2, when
    // n_kv is a multiple of 8 -- the group's K and V then come from HBM once, not once per head.
    const int rep = n_heads / n_kv, g = static_cast<int>(blockIdx.x) % n_kv;
    const int head = g * rep + static_cast<int>(blockIdx.x) / n_kv;
    // A decode step: the position in DecodeState.  A prompt chunk: row blockIdx.y of qkv / out
    // at position pos_first + blockIdx.y (every row's k and v already in the cache).
    const int pos = pos_first >= 0 ? pos_first + static_cast<int>(blockIdx.y) : st->pos, T = pos + 1;
    qkv += static_cast<size_t>(blockIdx.y) * qkv_stride;
    out += static_cast<size_t>(blockIdx.y) * out_stride;
    const int tid = static_cast<int>(threadIdx.x), lane = tid & (kWave - 1), wave = tid / kWave;
    float* ktile = sc + ((cap + 3) & ~3);   // tile rows of kst floats
    float* vtile = ktile + tile * kst;      // tile rows of hd floats
    float* dump = vtile + tile * hd;        // 4 floats: where stores past a tile's end go
    float* K = kc + static_cast<size_t>(g) * cap * hd;
    float* V = vc + static_cast<size_t>(g) * cap * hd;
    const bool one_round = T <= tile;

    // Load phase: this step's q, k, v, the RoPE factors and the first round's cached K and V
    // (positions < pos), every load issued before any store.  Thread i < hd / 2 rotates pair i
    // of q and k in registers; thread d < hd carries v[d].  The rotated k and v go to ks / vs,
    // into the tiles' row pos when the whole context is one round, and (the first workgroup of
    // the KV group) into the cache.
    {
        const int half = hd / 2;
        const int i = min(tid, half - 1), dv = min(tid, hd - 1);
        const int ia = interleaved ? 2 * i : i, ib = interleaved ? 2 * i + 1 : half + i;
        const float* qrow = qkv + static_cast<size_t>(head) * hd;
        const float* krow = qkv + static_cast<size_t>(n_heads + g) * hd;
        const float* cs = cos_tab + static_cast<size_t>(pos) * hd;
        const float* sn = sin_tab + static_cast<size_t>(pos) * hd;
        const float qa = qrow[ia], qb = qrow[ib], ka = krow[ia], kb = krow[ib];
        const float c0 = cs[i], s0 = sn[i], c1 = cs[half + i], s1 = sn[half + i];
        const float v0 = qkv[static_cast<size_t>(n_heads + n_kv + g) * hd + dv];
        const int first_cached = min(min(tile, T), pos);
        stage_tiles<true>(ktile, K, vtile, V, first_cached * hd, dump, hd / 4, kst);
        float q0, q1, k0, k1;
        if (interleaved) {
            rope_pair_interleaved(qa, qb, c0, s0, q0, q1);
            rope_pair_interleaved(ka, kb, c0, s0, k0, k1);
        } else {
            rope_pair_half(qa, qb, c0, s0, c1, s1, q0, q1);
            rope_pair_half(ka, kb, c0, s0, c1, s1, k0, k1);
        }
        const bool writer = head % rep == 0;
        if (tid < half) {
            qs[ia] = q0;
            qs[ib] = q1;
            ks[ia] = k0;
            ks[ib] = k1;
            if (one_round) {
                ktile[pos * kst + ia] = k0;
                ktile[pos * kst + ib] = k1;
            }
            if (writer) {
                K[static_cast<size_t>(pos) * hd + ia] = k0;
                K[static_cast<size_t>(pos) * hd + ib] = k1;
            }
        }
        if (tid < hd) {
            vs[tid] = v0;
            if (one_round) vtile[pos * hd + tid] = v0;
            if (writer) V[static_cast<size_t>(pos) * hd + tid] = v0;
        }
    }
    __syncthreads();

    // Scores, `tile` positions a round (one thread a position); rounds after the first restage
    // the K tile, position pos from ks.  Each thread keeps the maximum of the scores it writes
    // (and whether one is NaN or +inf) for the softmax.
    float mx = -__builtin_inff();
    int nonfinite = 0;
    for (int t0 = 0; t0 < T; t0 += tile) {
        const int tn = min(tile, T - t0);
        if (t0 > 0) {
            const int cached = min(tn, pos - t0);
            __syncthreads();  // the previous round's tile is consumed
            if (cached > 0)
                stage_tiles<false>(ktile, K + static_cast<size_t>(t0) * hd, nullptr, nullptr, cached * hd, dump,
                                   hd / 4, kst);
            if (cached < tn)
                for (int d = tid; d < hd; d += kAttnThreads) ktile[(pos - t0) * kst + d] = ks[d];
            __syncthreads();
        }
        for (int t = tid; t < tn; t += kAttnThreads) {
            const float v = position_score<HD>(qs, ktile + t * kst, hd, scale);
            sc[t0 + t] = v;
            const uint32_t u = __float_as_uint(v);
            nonfinite |= (u & 0x7fffffffu) > 0x7f800000u || u == 0x7f800000u;
            mx = fmaxf(mx, v);
        }
    }

    // Softmax over the T scores: the maximum (and whether any score is NaN or infinite; the
    // waves' partial maxima combined), the exponentials (the SIMD exp on full groups of 8, double
    // exp on the last T % 8), then the eight running double sums of the groups of 8 (lane j:
    // positions j, j+8, ... in order), added in lane order, then the tail's doubles, and 1 / sum.
    mx = group_max<kWave>(mx);
    nonfinite = group_sum_int<kWave>(nonfinite);
    if (lane == 0) {
        red_f[wave] = mx;
        red_i[wave] = nonfinite;
    }
    __syncthreads();
    mx = red_f[0];
    nonfinite = red_i[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
        mx = fmaxf(mx, red_f[w]);
        nonfinite |= red_i[w];
    }
    const bool nan_row = nonfinite || __float_as_uint(mx) == 0xff800000u;
    // The SIMD exp of the full groups of 8 by every thread; then, after a barrier, wave 0 runs the
    // eight double sums of those while the last eight threads (another wave) take the double exp of
    // the last T % 8 positions, which the sum needs only at its end; after a second barrier wave 0
    // adds them and forms 1 / sum.
    static_assert(kAttnThreads - 8 >= kWave, "the tail's threads are not in wave 0");
    const int n8 = T - T % 8;
    for (int t = tid; t < n8; t += kAttnThreads) sc[t] = exp_cody_waite(sc[t] - mx);
    __syncthreads();
    double sum = 0.0;
    if (wave == 0) {
        const double acc = lane < 8 ? strided_dsum(sc + lane, n8 / 8) : 0.0;
        double tsum = readlane_d(acc, 0);
#pragma unroll
        for (int k = 1; k < 8; ++k) tsum = tsum + readlane_d(acc, k);
        sum = 0.0 + tsum;
    } else if (tid >= kAttnThreads - 8) {
        const int j = tid - (kAttnThreads - 8);
        if (j < T - n8) {
            const double e = exp(static_cast<double>(sc[n8 + j] - mx));
            tail_e[j] = e;
            sc[n8 + j] = static_cast<float>(e);
        }
    }
    __syncthreads();
    if (wave == 0) {
        double tail[7];  // entries past T % 8 unused
#pragma unroll
        for (int j = 0; j < 7; ++j) tail[j] = tail_e[j];
#pragma unroll
        for (int j = 0; j < 7; ++j)
            if (j < T - n8) sum = sum + tail[j];
        if (lane == 0) inv_s = static_cast<float>(1.0 / sum);
    }
    __syncthreads();

    // p[t] = e[t] / sum as the product e[t] * (1 / sum) (NaN for a row with a NaN or infinite
    // score), in place, by every thread.
    const float inv = nan_row ? __builtin_nanf("") : inv_s;  // NaN * e = NaN for every position
    for (int t = tid; t < T; t += kAttnThreads) sc[t] = sc[t] * inv;
    __syncthreads();

    // out[d] = one fused chain over the positions in order of p[t] * V[t][d].
    float acc = 0.0f;
    const int d = tid;
    for (int t0 = 0; t0 < T; t0 += tile) {
        const int tn = min(tile, T - t0);
        if (t0 > 0) {
            const int cached = min(tn, pos - t0);
            __syncthreads();  // the previous tile is consumed
            if (cached > 0)
                stage_tiles<false>(vtile, V + static_cast<size_t>(t0) * hd, nullptr, nullptr, cached * hd, dump,
                                   hd / 4, hd);
            if (cached < tn)
                for (int e = tid; e < hd; e += kAttnThreads) vtile[(pos - t0) * hd + e] = vs[e];
            __syncthreads();
        }
        if (d < hd) acc = pv_chain<HD>(sc + t0, vtile + d, tn, hd, acc);
    }
    if (d < hd) out[static_cast<size_t>(head) * hd + d] = acc;
}

// Positions per round: the whole cache when it fits kMaxTile, else as many as the LDS budget
// leaves beside the scores (at least 16).
int attention_tile(int cap, int hd) {
    const size_t left = kAttnLdsBudget / 4 - static_cast<size_t>((cap + 3) & ~3) - 4;  // 4: the spare slot
    // (a multiple of 8, so that every round's p starts 16-byte aligned)
    const int fit = static_cast<int>(left / static_cast<size_t>(k_stride(hd) + hd)) & ~7;
    return std::max(16, std::min({kMaxTile, cap, fit}));
}
size_t attention_lds(int cap, int hd) {
    return (static_cast<size_t>((cap + 3) & ~3) + static_cast<size_t>(attention_tile(cap, hd)) * (k_stride(hd) + hd) +
            4) *
           4;
}

// The instantiation for a head_dim: 64 and 128 unrolled, any other the run-time loop.
using AttentionFn = decltype(&attention_kernel<0>);
AttentionFn attention_for(int hd) {
    return hd == 64 ? attention_kernel<64> : hd == 128 ? attention_kernel<128> : attention_kernel<0>;
}

// RoPE of one head of hd values in place in LDS (hd / 2 threads).
__device__ __forceinline__ void rope_head_lds(float* v, const float* cs, const float* sn, int hd, int interleaved) {
    const int half = hd / 2, i = threadIdx.x;
    if (i < half) {
        if (interleaved) {
            float o0, o1;
            rope_pair_interleaved(v[2 * i], v[2 * i + 1], cs[i], sn[i], o0, o1);
            v[2 * i] = o0;
            v[2 * i + 1] = o1;
        } else {
            float o0, o1;
            rope_pair_half(v[i], v[half + i], cs[i], sn[i], cs[half + i], sn[half + i], o0, o1);
            v[i] = o0;
            v[half + i] = o1;
        }
    }
}

// Prompt chunk: k = rope(k) and v of rows p < gridDim.y into the cache at pos_first + p, for KV
// group blockIdx.x -- the values attention_kernel writes for a decode step (same operations),
// so that every row's attention can read the positions before it from the cache.
__global__ __launch_bounds__(kRopeKvThreads) void rope_kv_kernel(const float* __restrict__ qkv, int qkv_stride,
                                                               const float* __restrict__ cos_tab,
                                                               const float* __restrict__ sin_tab, int interleaved,
                                                               float* __restrict__ kc, float* __restrict__ vc,
                                                               int n_heads, int n_kv, int hd, int cap, int pos_first) {
    __shared__ float ks[kHeadMax];
    const int g = blockIdx.x, p = blockIdx.y, pos = pos_first + p;
    const float* row = qkv + static_cast<size_t>(p) * qkv_stride;
    const int d = threadIdx.x;
    float v0 = 0.0f;
    if (d < hd) {
        ks[d] = row[static_cast<size_t>(n_heads + g) * hd + d];
        v0 = row[static_cast<size_t>(n_heads + n_kv + g) * hd + d];
    }
    __syncthreads();
    rope_head_lds(ks, cos_tab + static_cast<size_t>(pos) * hd, sin_tab + static_cast<size_t>(pos) * hd, hd, interleaved);
    __syncthreads();
    if (d < hd) {
        const size_t at = (static_cast<size_t>(g) * cap + pos) * hd + d;
        kc[at] = ks[d];
        vc[at] = v0;
    }
}

// Prompt chunk: m[p][n] = silu(gate[p][n]) * up[p][n] from gu rows of 2 ffn values -- gate n and
// up n at 2n and 2n+1 (interleaved weights) or at n and ffn + n -- the decode step's operations.
__global__ void silu_mul_rows_kernel(const float* __restrict__ gu, int rows, int ffn, int interleaved,
                                     float* __restrict__ m) {
    const long long total = static_cast<long long>(rows) * ffn;
    for (long long e = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; e < total;
         e += static_cast<long long>(gridDim.x) * blockDim.x) {
        const long long p = e / ffn, n = e - p * ffn;
        const float* r = gu + p * 2 * ffn;
        const float gate = interleaved ? r[2 * n] : r[n], up = interleaved ? r[2 * n + 1] : r[ffn + n];
        m[e] = silu_ref(gate) * up;
    }
}

// m = silu(g) * u (llama.py:434: sk.silu(gate) * up, two float32 results multiplied), SiLU as
// the reference's SIMD tables compute it.
__global__ void silu_mul_kernel(const float* __restrict__ gu, int ffn, float* __restrict__ m) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < ffn; i += gridDim.x * blockDim.x)
        m[i] = silu_ref(gu[i]) * gu[ffn + i];
}

// np.argmax semantics: the first index of the maximum; a NaN counts as the maximum (the first
// NaN wins).
__device__ __forceinline__ bool better(float a, int ia, float b, int ib) {
    const bool an = a != a, bn = b != b;
    if (an || bn) return an && (!bn || ia < ib);
    return a > b || (a == b && ia < ib);
}

// Greedy next token in two stages: kArgmaxParts workgroups take contiguous slices of the
// logits, then one wave merges their (value, index) candidates -- np.argmax's rule is
// preserved because `better` breaks ties by the smaller index -- writes tokens[pos + 1] (only
// past the given prompt) and advances the position.
constexpr int kArgmaxParts = 128;
constexpr int kArgmaxThreads = 256;

__device__ __forceinline__ void argmax_wave(float& v, int& idx) {
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, kWave);
        const int oi = __shfl_xor(idx, off, kWave);
        if (better(ov, oi, v, idx)) {
            v = ov;
            idx = oi;
        }
    }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_part_kernel(const float* __restrict__ logits, int n,
                                                                     float* __restrict__ pv, int* __restrict__ pi) {
    __shared__ float bv[kArgmaxThreads / kWave];
    __shared__ int bi[kArgmaxThreads / kWave];
    const int chunk = (n + gridDim.x - 1) / gridDim.x;
    const int lo = blockIdx.x * chunk, hi = min(n, lo + chunk);
    float v = -__builtin_inff();
    int idx = 0x7fffffff;
    for (int i = lo + threadIdx.x; i < hi; i += kArgmaxThreads) {
        const float c = logits[i];
        if (better(c, i, v, idx)) {
            v = c;
            idx = i;
        }
    }
    argmax_wave(v, idx);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    if (lane == 0) {
        bv[wave] = v;
        bi[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kArgmaxThreads / kWave; ++w)
            if (better(bv[w], bi[w], v, idx)) {
                v = bv[w];
                idx = bi[w];
            }
        pv[blockIdx.x] = v;
        pi[blockIdx.x] = idx;
    }
}

// ... and x = the embedding row of the next step's token (the prompt's next token, or the
// argmax past the prompt), so that a decode step that follows needs no embedding launch.
__global__ __launch_bounds__(kWave) void argmax_final_kernel(const float* __restrict__ pv, const int* __restrict__ pi,
                                                             int parts, int n, int* __restrict__ tokens, int cap,
                                                             DecodeState* __restrict__ st, const uint8_t* __restrict__ E,
                                                             int etype, int hidden, float* __restrict__ x) {
    const int p = st->pos, n_prompt = st->n_prompt;  // read by every lane before lane 0 advances pos
    float v = -__builtin_inff();
    int idx = 0x7fffffff;
    for (int b = threadIdx.x; b < parts; b += kWave)
        if (better(pv[b], pi[b], v, idx)) {
            v = pv[b];
            idx = pi[b];
        }
    argmax_wave(v, idx);  // every lane holds the result
    if (idx < 0 || idx >= n) idx = 0;  // n == 0 cannot happen (vocab > 0)
    if (threadIdx.x == 0) {
        if (p + 1 >= n_prompt && p + 1 <= cap) tokens[p + 1] = idx;
        st->pos = p + 1;
    }
    if (p + 1 <= cap) embed_row(E, etype, hidden, n, p + 1 < n_prompt ? tokens[p + 1] : idx, x);
}

__global__ void advance_kernel(DecodeState* st) {
    if (threadIdx.x == 0) st->pos = st->pos + 1;
}

// ─── the model ──────────────────────────────────────────────────────────────

int type_block_bytes(int type) { return type == kGgmlQ4_0 ? kQ4_0Bytes : type == kGgmlQ8_0 ? kQ8_0Bytes : 0; }

size_t matrix_bytes(int type, int rows, int cols) {
    if (type == kGgmlF32) return static_cast<size_t>(rows) * cols * 4;
    return static_cast<size_t>(rows) * (cols / 32) * type_block_bytes(type);
}

struct Mat {
    uint8_t* p = nullptr;
    int type = kGgmlQ4_0, rows = 0, cols = 0;
    size_t bytes() const { return matrix_bytes(type, rows, cols); }
    size_t row_bytes() const { return rows ? bytes() / rows : 0; }
};

struct Layer {
    float* attn_norm = nullptr;
    float* ffn_norm = nullptr;
    Mat qkv, o, gateup, down;
};

// Section marks of a profiled (eager) step: an event recorded at each section start; the time
// up to the next mark is the section's.  Sections: see smk_llama_step_profile.
enum Section { kEmbed = 0, kRms, kGemvQkv, kRopeKv, kAttention, kGemvO, kGemvGateUp, kSiluMul, kGemvDown,
               kLmHead, kArgmax, kSections };

struct Marks {
    std::vector<hipEvent_t> ev;
    std::vector<int> id;
    hipError_t mark(hipStream_t s, int section) {
        if (id.size() == ev.size()) {
            hipEvent_t e;
            if (const hipError_t r = hipEventCreate(&e); r != hipSuccess) return r;
            ev.push_back(e);
        }
        id.push_back(section);
        return hipEventRecord(ev[id.size() - 1], s);
    }
};

struct Model {
    smk_llama_config cfg{};
    hipStream_t stream = nullptr;
    Mat embed, head;
    bool tied = true;
    float* out_norm = nullptr;
    std::vector<Layer> layers;
    std::vector<void*> allocs;
    // activations
    float *x = nullptr, *h = nullptr, *qkv = nullptr, *attn = nullptr, *gu = nullptr, *m = nullptr,
          *logits = nullptr;
    DecodeState* st = nullptr;
    float* part_v = nullptr;     // argmax candidates
    int* part_i = nullptr;
    int* host_pinned = nullptr;  // staging for tokens and state
    // per capacity
    int capacity = 0;
    int pos = 0;
    int* tokens = nullptr;
    float *kc = nullptr, *vc = nullptr, *cos_tab = nullptr, *sin_tab = nullptr;
    hipGraphExec_t g_logits = nullptr, g_plain = nullptr;
    hipGraphExec_t g_next = nullptr;  // a logits step whose embedding the previous step's argmax wrote
    std::vector<unsigned> loaded;  // bit per tensor per layer
    bool fuse_norm = false;        // Q4_0 GEMVs normalize x themselves
    bool fuse_silu = false;        // gate/up rows interleaved; the GEMV writes silu(gate) * up
    hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
    Marks marks;
    uint64_t weight_bytes = 0;
    // prompt chunks (generate): rows per chunk (< 2: one graph step per prompt token) and the
    // chunk's activations, row-major [rows][width]
    int prefill_rows = 64;
    int batch_rows = 0;
    float *bx = nullptr, *bh = nullptr, *bqkv = nullptr, *battn = nullptr, *bgu = nullptr, *bm = nullptr;

    int q_rows() const { return cfg.n_heads * cfg.head_dim; }
    int kv_rows() const { return cfg.n_kv_heads * cfg.head_dim; }
};

hipError_t dalloc(Model& md, void** p, size_t bytes) {
    *p = nullptr;
    const hipError_t e = hipMalloc(p, std::max<size_t>(bytes, 256));
    if (e == hipSuccess) md.allocs.push_back(*p);
    return e;
}

void free_capacity(Model& md) {
    if (md.g_logits) (void)hipGraphExecDestroy(md.g_logits);
    if (md.g_plain) (void)hipGraphExecDestroy(md.g_plain);
    if (md.g_next) (void)hipGraphExecDestroy(md.g_next);
    md.g_logits = md.g_plain = md.g_next = nullptr;
    for (void* p : {static_cast<void*>(md.tokens), static_cast<void*>(md.kc), static_cast<void*>(md.vc),
                    static_cast<void*>(md.cos_tab), static_cast<void*>(md.sin_tab)})
        if (p) (void)hipFree(p);
    md.tokens = nullptr;
    md.kc = md.vc = md.cos_tab = md.sin_tab = nullptr;
    md.capacity = 0;
}

// y (+)= RMSNorm(x, nw) . W^T: the Q4_0 GEMV normalizes x in its own prologue when the model
// allows it (fuse_norm), else the RMSNorm kernel writes h first.
hipError_t gemv(const Mat& W, const float* x, float* y, bool accumulate, hipStream_t s);

hipError_t gemv_normed(const Model& md, const Mat& W, const float* x, const float* nw, float* h, float* y,
                       bool accumulate, bool silu_pairs = false) {
    GemvTuning t;
    t.accumulate = accumulate ? 1 : 0;
    t.silu_pairs = silu_pairs ? 1 : 0;
    t.stream_weights = 1;
    if (md.fuse_norm && W.type == kGgmlQ4_0) {
        t.norm_w = nw;
        t.norm_eps = md.cfg.rms_eps;
        return gemv_quant(kQ4_0Bytes, 1, W.rows, W.cols, x, W.cols, W.p, y, W.rows, md.stream, &t);
    }
    if (const hipError_t e = rms_norm(x, nw, h, 1, md.cfg.hidden, md.cfg.rms_eps, md.stream); e != hipSuccess) return e;
    if (silu_pairs) return gemv_quant(kQ4_0Bytes, 1, W.rows, W.cols, h, W.cols, W.p, y, W.rows, md.stream, &t);
    return gemv(W, h, y, accumulate, md.stream);
}

hipError_t gemv(const Mat& W, const float* x, float* y, bool accumulate, hipStream_t s) {
    if (W.type == kGgmlF32)
        return gemm_tb(0, 1, W.rows, W.cols, 1.0f, x, W.cols, W.p, W.cols, accumulate ? 1.0f : 0.0f, y, W.rows, s);
    GemvTuning t;
    t.accumulate = accumulate ? 1 : 0;
    t.stream_weights = 1;
    return gemv_quant(type_block_bytes(W.type), 1, W.rows, W.cols, x, W.cols, W.p, y, W.rows, s, &t);
}

// Enqueue one decode step (the body every graph captures).
#define SMK_MARK(section)                                                         \
    do {                                                                          \
        if (mk)                                                                   \
            if (const hipError_t e_ = mk->mark(s, section); e_ != hipSuccess) return e_; \
    } while (0)

// embed = false: x already holds the step's embedding row (the previous step's argmax wrote it).
hipError_t enqueue_step(Model& md, bool with_logits, Marks* mk = nullptr, bool embed = true) {
    const smk_llama_config& c = md.cfg;
    hipStream_t s = md.stream;
    const int nh = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim;
    SMK_MARK(kEmbed);
    if (embed) {
        hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(256), 0, s, md.embed.p, md.embed.type, c.hidden, c.vocab,
                           md.tokens, md.st, md.x);
        if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    const size_t layer_kv = static_cast<size_t>(nkv) * md.capacity * hd;
    const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(hd)));
    for (int l = 0; l < c.n_layers; ++l) {
        const Layer& L = md.layers[l];
        float* kc = md.kc + l * layer_kv;
        float* vc = md.vc + l * layer_kv;
        SMK_MARK(kGemvQkv);
        hipError_t e = gemv_normed(md, L.qkv, md.x, L.attn_norm, md.h, md.qkv, false);
        if (e != hipSuccess) return e;
        SMK_MARK(kAttention);
        hipLaunchKernelGGL(attention_for(hd), dim3(nh), dim3(kAttnThreads), attention_lds(md.capacity, hd), s,
                           md.qkv, md.cos_tab, md.sin_tab, c.rope_interleaved, kc, vc, nh, nkv, hd, md.capacity,
                           scale, attention_tile(md.capacity, hd), md.st, md.attn, -1, 0, 0);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        SMK_MARK(kGemvO);
        if ((e = gemv(L.o, md.attn, md.x, true, s)) != hipSuccess) return e;
        SMK_MARK(kGemvGateUp);
        if (md.fuse_silu) {
            if ((e = gemv_normed(md, L.gateup, md.x, L.ffn_norm, md.h, md.m, false, true)) != hipSuccess) return e;
        } else {
            if ((e = gemv_normed(md, L.gateup, md.x, L.ffn_norm, md.h, md.gu, false)) != hipSuccess) return e;
            SMK_MARK(kSiluMul);
            hipLaunchKernelGGL(silu_mul_kernel, dim3((c.ffn + 255) / 256), dim3(256), 0, s, md.gu, c.ffn, md.m);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        SMK_MARK(kGemvDown);
        if ((e = gemv(L.down, md.m, md.x, true, s)) != hipSuccess) return e;
    }
    if (!with_logits) {
        SMK_MARK(kArgmax);
        hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, s, md.st);
        return hipGetLastError();
    }
    SMK_MARK(kLmHead);
    if (md.fuse_norm && md.head.type == kGgmlQ4_0 && c.hidden == 2048) {
        // One launch: the lm_head's tiled kernel normalizes x in its prologue (width 2048).
        if (const hipError_t e = gemv_normed(md, md.head, md.x, md.out_norm, md.h, md.logits, false); e != hipSuccess)
            return e;
    } else {
        // The final RMSNorm as a kernel of its own, then the plain lm_head product: a plain Q4_0
        // product of this many rows takes the K-chunk tiled kernel, which the fused-norm form
        // takes only at width 2048 (same bits either way).
        if (const hipError_t e = rms_norm(md.x, md.out_norm, md.h, 1, c.hidden, c.rms_eps, s); e != hipSuccess)
            return e;
        if (const hipError_t e = gemv(md.head, md.h, md.logits, false, s); e != hipSuccess) return e;
    }
    SMK_MARK(kArgmax);
    hipLaunchKernelGGL(argmax_part_kernel, dim3(kArgmaxParts), dim3(kArgmaxThreads), 0, s, md.logits, c.vocab,
                       md.part_v, md.part_i);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kWave), 0, s, md.part_v, md.part_i, kArgmaxParts, c.vocab,
                       md.tokens, md.capacity, md.st, md.embed.p, md.embed.type, c.hidden, md.x);
    return hipGetLastError();
}
#undef SMK_MARK

// The prompt in chunks of rows (examples/llama/llama.py:491-492 runs it token by token): every
// matrix product takes all rows of the chunk at once (the matrix-core Q4_0 kernel), RMSNorm and
// SiLU run over the rows, rope_kv_kernel fills the chunk's cache positions, and one attention
// launch covers (head, row).  Each row's arithmetic is the decode step's, so the cache and the
// first generated token equal the token-by-token run bit for bit.  Needs quantized matrices (the
// batched Q4_0 / Q8_0 products equal their one-row calls; the FP32 ones are not pinned to).
bool chunked_prefill_ok(const Model& md) {
    return md.prefill_rows >= 2 && (md.cfg.matrix_type == kGgmlQ4_0 || md.cfg.matrix_type == kGgmlQ8_0);
}

hipError_t batch_buffers(Model& md, int rows) {
    if (md.batch_rows >= rows) return hipSuccess;
    for (float** p : {&md.bx, &md.bh, &md.bqkv, &md.battn, &md.bgu, &md.bm}) {
        if (*p) {
            md.allocs.erase(std::remove(md.allocs.begin(), md.allocs.end(), static_cast<void*>(*p)), md.allocs.end());
            (void)hipFree(*p);
            *p = nullptr;
        }
    }
    md.batch_rows = 0;
    const smk_llama_config& c = md.cfg;
    const size_t r = static_cast<size_t>(rows) * 4;
    const size_t qkv_rows = static_cast<size_t>(md.q_rows() + 2 * md.kv_rows());
    struct Want { float** p; size_t bytes; };
    for (const Want& w : {Want{&md.bx, r * c.hidden}, Want{&md.bh, r * c.hidden}, Want{&md.bqkv, r * qkv_rows},
                          Want{&md.battn, r * md.q_rows()}, Want{&md.bgu, r * 2 * c.ffn}, Want{&md.bm, r * c.ffn}})
        if (const hipError_t e = dalloc(md, reinterpret_cast<void**>(w.p), w.bytes); e != hipSuccess) return e;
    md.batch_rows = rows;
    return hipSuccess;
}

// Prompt rows [first, first + P): the KV cache at those positions; with logits, also the last
// row's logits and argmax (DecodeState.pos must then be first + P - 1: the argmax writes
// tokens[first + P] and advances it).
hipError_t enqueue_prompt_chunk(Model& md, int first, int P, bool with_logits) {
    const smk_llama_config& c = md.cfg;
    hipStream_t s = md.stream;
    const int nh = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim, H = c.hidden;
    const int qkv_rows = md.q_rows() + 2 * md.kv_rows();
    const int bb = type_block_bytes(c.matrix_type);
    hipLaunchKernelGGL(embed_rows_kernel, dim3(P), dim3(256), 0, s, md.embed.p, md.embed.type, H, c.vocab,
                       md.tokens + first, md.bx);
    if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    const size_t layer_kv = static_cast<size_t>(nkv) * md.capacity * hd;
    const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(hd)));
    GemvTuning plain, acc;
    acc.accumulate = 1;
    for (int l = 0; l < c.n_layers; ++l) {
        const Layer& L = md.layers[l];
        float* kc = md.kc + l * layer_kv;
        float* vc = md.vc + l * layer_kv;
        hipError_t e = rms_norm(md.bx, L.attn_norm, md.bh, P, H, c.rms_eps, s);
        if (e == hipSuccess) e = gemv_quant(bb, P, qkv_rows, H, md.bh, H, L.qkv.p, md.bqkv, qkv_rows, s, &plain);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(rope_kv_kernel, dim3(nkv, P), dim3(kRopeKvThreads), 0, s, md.bqkv, qkv_rows, md.cos_tab,
                           md.sin_tab, c.rope_interleaved, kc, vc, nh, nkv, hd, md.capacity, first);
        hipLaunchKernelGGL(attention_for(hd), dim3(nh, P), dim3(kAttnThreads), attention_lds(md.capacity, hd), s,
                           md.bqkv, md.cos_tab, md.sin_tab, c.rope_interleaved, kc, vc, nh, nkv, hd, md.capacity,
                           scale, attention_tile(md.capacity, hd), md.st, md.battn, first, qkv_rows, md.q_rows());
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if ((e = gemv_quant(bb, P, H, md.q_rows(), md.battn, md.q_rows(), L.o.p, md.bx, H, s, &acc)) != hipSuccess)
            return e;
        if ((e = rms_norm(md.bx, L.ffn_norm, md.bh, P, H, c.rms_eps, s)) != hipSuccess) return e;
        if ((e = gemv_quant(bb, P, 2 * c.ffn, H, md.bh, H, L.gateup.p, md.bgu, 2 * c.ffn, s, &plain)) != hipSuccess)
            return e;
        const long long total = static_cast<long long>(P) * c.ffn;
        hipLaunchKernelGGL(silu_mul_rows_kernel, dim3(static_cast<int>(std::min<long long>((total + 255) / 256, 4096))),
                           dim3(256), 0, s, md.bgu, P, c.ffn, md.fuse_silu ? 1 : 0, md.bm);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if ((e = gemv_quant(bb, P, H, c.ffn, md.bm, c.ffn, L.down.p, md.bx, H, s, &acc)) != hipSuccess) return e;
    }
    if (!with_logits) return hipSuccess;
    const float* xl = md.bx + static_cast<size_t>(P - 1) * H;
    if (const hipError_t e = gemv_normed(md, md.head, xl, md.out_norm, md.h, md.logits, false); e != hipSuccess)
        return e;
    hipLaunchKernelGGL(argmax_part_kernel, dim3(kArgmaxParts), dim3(kArgmaxThreads), 0, s, md.logits, c.vocab,
                       md.part_v, md.part_i);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kWave), 0, s, md.part_v, md.part_i, kArgmaxParts, c.vocab,
                       md.tokens, md.capacity, md.st, md.embed.p, md.embed.type, c.hidden, md.x);
    return hipGetLastError();
}

hipError_t capture(Model& md, bool with_logits, hipGraphExec_t* out, bool embed = true) {
    hipError_t e = hipStreamBeginCapture(md.stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return e;
    const hipError_t body = enqueue_step(md, with_logits, nullptr, embed);
    hipGraph_t graph = nullptr;
    e = hipStreamEndCapture(md.stream, &graph);
    if (body != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return body;
    }
    if (e != hipSuccess) return e;
    e = hipGraphInstantiate(out, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    return e;
}

// Tensor ids of smk_llama_set_tensor.
enum { T_EMBD = 0, T_OUT_NORM, T_OUTPUT, T_ATTN_NORM, T_Q, T_K, T_V, T_O, T_FFN_NORM, T_GATE, T_UP, T_DOWN, T_COUNT };

bool all_loaded(const Model& md, std::string* missing) {
    const int L = md.cfg.n_layers;
    if (!(md.loaded[0] & (1u << T_EMBD))) return *missing = "token_embd", false;
    if (!(md.loaded[0] & (1u << T_OUT_NORM))) return *missing = "output_norm", false;
    if (!md.tied && !(md.loaded[0] & (1u << T_OUTPUT))) return *missing = "output", false;
    for (int l = 0; l < L; ++l)
        for (int t = T_ATTN_NORM; t < T_COUNT; ++t)
            if (!(md.loaded[1 + l] & (1u << t))) return *missing = "layer " + std::to_string(l) + " tensor " + std::to_string(t), false;
    return true;
}

}  // namespace
}  // namespace smk

using namespace smk;
using namespace smk::abi;

extern "C" {

int smk_llama_create(const smk_llama_config* cfg, void** model) {
    if (!cfg || !model) return fail(SMK_ERR_ARGUMENT, "null argument");
    *model = nullptr;
    const smk_llama_config& c = *cfg;
    if (c.n_layers <= 0 || c.hidden <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 || c.ffn <= 0 ||
        c.vocab <= 0)
        return fail(SMK_ERR_ARGUMENT, "every dimension must be positive");
    if (c.n_heads % c.n_kv_heads) return fail(SMK_ERR_ARGUMENT, "n_heads must be a multiple of n_kv_heads");
    if (c.head_dim % 4 || c.head_dim > 256) return fail(SMK_ERR_ARGUMENT, "head_dim must be a multiple of 4 and <= 256");
    if (c.hidden % 32 || c.ffn % 32 || (c.n_heads * c.head_dim) % 32)
        return fail(SMK_ERR_ARGUMENT, "hidden, ffn and n_heads*head_dim must be multiples of 32");
    for (int t : {c.matrix_type, c.embed_type})
        if (t != kGgmlF32 && t != kGgmlQ4_0 && t != kGgmlQ8_0)
            return fail(SMK_ERR_ARGUMENT, "weight types: 0 (F32), 2 (Q4_0) or 8 (Q8_0)");
    if (c.head_type != -1 && c.head_type != kGgmlF32 && c.head_type != kGgmlQ4_0 && c.head_type != kGgmlQ8_0)
        return fail(SMK_ERR_ARGUMENT, "head_type: -1 (tied), 0, 2 or 8");
    if (const int rc = use_device()) return rc;
    auto* md = new Model();
    md->cfg = c;
    md->tied = c.head_type == -1;
    md->loaded.assign(1 + c.n_layers, 0u);
    auto cleanup = [&](hipError_t e, const char* what) {
        for (void* p : md->allocs) (void)hipFree(p);
        if (md->stream) (void)hipStreamDestroy(md->stream);
        if (md->host_pinned) (void)hipHostFree(md->host_pinned);
        for (hipEvent_t& ev : md->ev)
            if (ev) (void)hipEventDestroy(ev);
        delete md;
        return hip_fail(e, what);
    };
    hipError_t e = hipStreamCreateWithFlags(&md->stream, hipStreamNonBlocking);
    if (e != hipSuccess) return cleanup(e, "stream");
    for (hipEvent_t& ev : md->ev)
        if ((e = hipEventCreate(&ev)) != hipSuccess) return cleanup(e, "event");
    if ((e = hipHostMalloc(reinterpret_cast<void**>(&md->host_pinned), 4096, hipHostMallocDefault)) != hipSuccess)
        return cleanup(e, "pinned staging");
    const int qkv_rows = md->q_rows() + 2 * md->kv_rows();
    md->embed = {nullptr, c.embed_type, c.vocab, c.hidden};
    md->head = md->tied ? md->embed : Mat{nullptr, c.head_type, c.vocab, c.hidden};
    struct Want { void** p; size_t bytes; };
    std::vector<Want> want = {
        {reinterpret_cast<void**>(&md->embed.p), md->embed.bytes()},
        {reinterpret_cast<void**>(&md->out_norm), static_cast<size_t>(c.hidden) * 4},
        {reinterpret_cast<void**>(&md->x), static_cast<size_t>(c.hidden) * 4},
        {reinterpret_cast<void**>(&md->h), static_cast<size_t>(std::max(c.hidden, md->q_rows())) * 4},
        {reinterpret_cast<void**>(&md->qkv), static_cast<size_t>(qkv_rows) * 4},
        {reinterpret_cast<void**>(&md->attn), static_cast<size_t>(md->q_rows()) * 4},
        {reinterpret_cast<void**>(&md->gu), static_cast<size_t>(2 * c.ffn) * 4},
        {reinterpret_cast<void**>(&md->m), static_cast<size_t>(c.ffn) * 4},
        {reinterpret_cast<void**>(&md->logits), static_cast<size_t>(c.vocab) * 4},
        {reinterpret_cast<void**>(&md->st), sizeof(DecodeState)},
        {reinterpret_cast<void**>(&md->part_v), static_cast<size_t>(kArgmaxParts) * 4},
        {reinterpret_cast<void**>(&md->part_i), static_cast<size_t>(kArgmaxParts) * 4},
    };
    if (!md->tied) want.push_back({reinterpret_cast<void**>(&md->head.p), md->head.bytes()});
    md->layers.resize(c.n_layers);
    for (Layer& L : md->layers) {
        L.qkv = {nullptr, c.matrix_type, qkv_rows, c.hidden};
        L.o = {nullptr, c.matrix_type, c.hidden, md->q_rows()};
        L.gateup = {nullptr, c.matrix_type, 2 * c.ffn, c.hidden};
        L.down = {nullptr, c.matrix_type, c.hidden, c.ffn};
        want.push_back({reinterpret_cast<void**>(&L.attn_norm), static_cast<size_t>(c.hidden) * 4});
        want.push_back({reinterpret_cast<void**>(&L.ffn_norm), static_cast<size_t>(c.hidden) * 4});
        for (Mat* M : {&L.qkv, &L.o, &L.gateup, &L.down}) want.push_back({reinterpret_cast<void**>(&M->p), M->bytes()});
    }
    for (const Want& w : want)
        if ((e = dalloc(*md, w.p, w.bytes)) != hipSuccess) return cleanup(e, "model allocation");
    if (md->tied) md->head = md->embed;
    {
        const int depth = uniform_depth(c.hidden);
        md->fuse_norm = c.matrix_type == kGgmlQ4_0 && c.hidden <= 8192 && c.hidden % 64 == 0 &&
                        uniform_equal_leaves(c.hidden, depth) &&
                        (8 << depth) <= 1024 && (md->q_rows() + 2 * md->kv_rows()) % 2 == 0 && c.vocab % 2 == 0;
        md->fuse_silu = c.matrix_type == kGgmlQ4_0 && c.hidden % 64 == 0;
    }
    md->weight_bytes = md->head.bytes();
    for (const Layer& L : md->layers) md->weight_bytes += L.qkv.bytes() + L.o.bytes() + L.gateup.bytes() + L.down.bytes();
    *model = md;
    return ok();
}

int smk_llama_destroy(void* model) {
    if (!model) return ok();
    auto* md = static_cast<Model*>(model);
    if (const int rc = use_device()) return rc;
    (void)hipStreamSynchronize(md->stream);
    free_capacity(*md);
    for (void* p : md->allocs) (void)hipFree(p);
    for (hipEvent_t& ev : md->ev)
        if (ev) (void)hipEventDestroy(ev);
    for (hipEvent_t ev : md->marks.ev) (void)hipEventDestroy(ev);
    if (md->host_pinned) (void)hipHostFree(md->host_pinned);
    (void)hipStreamDestroy(md->stream);
    delete md;
    return ok();
}

int smk_llama_set_tensor(void* model, int tensor, int layer, const void* host, size_t nbytes) {
    if (!model || !host) return fail(SMK_ERR_ARGUMENT, "null argument");
    auto* md = static_cast<Model*>(model);
    const smk_llama_config& c = md->cfg;
    const bool per_layer = tensor >= T_ATTN_NORM && tensor < T_COUNT;
    if (tensor < 0 || tensor >= T_COUNT) return fail(SMK_ERR_ARGUMENT, "unknown tensor id");
    if (per_layer && (layer < 0 || layer >= c.n_layers)) return fail(SMK_ERR_ARGUMENT, "layer out of range");
    if (tensor == T_OUTPUT && md->tied) return fail(SMK_ERR_ARGUMENT, "output.weight given but head_type is -1 (tied)");
    if (const int rc = use_device()) return rc;
    void* dst = nullptr;
    size_t want = 0;
    if (tensor == T_EMBD) {
        dst = md->embed.p;
        want = md->embed.bytes();
    } else if (tensor == T_OUT_NORM) {
        dst = md->out_norm;
        want = static_cast<size_t>(c.hidden) * 4;
    } else if (tensor == T_OUTPUT) {
        dst = md->head.p;
        want = md->head.bytes();
    } else {
        Layer& L = md->layers[layer];
        const int qr = md->q_rows(), kr = md->kv_rows();
        switch (tensor) {
            case T_ATTN_NORM: dst = L.attn_norm; want = static_cast<size_t>(c.hidden) * 4; break;
            case T_FFN_NORM: dst = L.ffn_norm; want = static_cast<size_t>(c.hidden) * 4; break;
            case T_Q: dst = L.qkv.p; want = static_cast<size_t>(qr) * L.qkv.row_bytes(); break;
            case T_K: dst = L.qkv.p + static_cast<size_t>(qr) * L.qkv.row_bytes(); want = static_cast<size_t>(kr) * L.qkv.row_bytes(); break;
            case T_V: dst = L.qkv.p + static_cast<size_t>(qr + kr) * L.qkv.row_bytes(); want = static_cast<size_t>(kr) * L.qkv.row_bytes(); break;
            case T_O: dst = L.o.p; want = L.o.bytes(); break;
            case T_GATE:
            case T_UP: {
                // Gate rows then up rows; interleaved (gate_n, up_n) when the GEMV fuses the SiLU.
                const size_t rb = L.gateup.row_bytes();
                want = static_cast<size_t>(c.ffn) * rb;
                if (nbytes != want) break;
                if (md->fuse_silu) {
                    SMK_HIP(hipMemcpy2D(L.gateup.p + (tensor == T_UP ? rb : 0), 2 * rb, host, rb, rb, c.ffn,
                                        hipMemcpyHostToDevice),
                            "tensor upload");
                } else {
                    SMK_HIP(hipMemcpy(L.gateup.p + (tensor == T_UP ? c.ffn * rb : 0), host, want, hipMemcpyHostToDevice),
                            "tensor upload");
                }
                md->loaded[1 + layer] |= 1u << tensor;
                return ok();
            }
            case T_DOWN: dst = L.down.p; want = L.down.bytes(); break;
        }
    }
    if (nbytes != want)
        return fail(SMK_ERR_ARGUMENT, "tensor " + std::to_string(tensor) + ": " + std::to_string(nbytes) +
                                          " bytes given, " + std::to_string(want) + " expected for its shape and type");
    SMK_HIP(hipMemcpy(dst, host, nbytes, hipMemcpyHostToDevice), "tensor upload");
    md->loaded[per_layer ? 1 + layer : 0] |= 1u << tensor;
    return ok();
}

int smk_llama_reset(void* model, int capacity, const float* cos_table, const float* sin_table) {
    if (!model || !cos_table || !sin_table) return fail(SMK_ERR_ARGUMENT, "null argument");
    auto* md = static_cast<Model*>(model);
    if (capacity <= 0 || capacity > kMaxCapacity)
        return fail(SMK_ERR_ARGUMENT, "capacity must be in [1, " + std::to_string(kMaxCapacity) + "]");
    std::string missing;
    if (!all_loaded(*md, &missing)) return fail(SMK_ERR_ARGUMENT, "tensor not loaded: " + missing);
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipStreamSynchronize(md->stream), "synchronize");
    const smk_llama_config& c = md->cfg;
    const size_t kv = static_cast<size_t>(c.n_layers) * c.n_kv_heads * capacity * c.head_dim * 4;
    const size_t tab = static_cast<size_t>(capacity) * c.head_dim * 4;
    if (capacity != md->capacity) {
        free_capacity(*md);
        SMK_HIP(hipMalloc(reinterpret_cast<void**>(&md->tokens), static_cast<size_t>(capacity + 1) * 4), "tokens");
        SMK_HIP(hipMalloc(reinterpret_cast<void**>(&md->kc), kv), "k cache");
        SMK_HIP(hipMalloc(reinterpret_cast<void**>(&md->vc), kv), "v cache");
        SMK_HIP(hipMalloc(reinterpret_cast<void**>(&md->cos_tab), tab), "cos table");
        SMK_HIP(hipMalloc(reinterpret_cast<void**>(&md->sin_tab), tab), "sin table");
        md->capacity = capacity;
    }
    SMK_HIP(hipMemsetAsync(md->kc, 0, kv, md->stream), "k cache clear");
    SMK_HIP(hipMemsetAsync(md->vc, 0, kv, md->stream), "v cache clear");
    SMK_HIP(hipMemsetAsync(md->tokens, 0, static_cast<size_t>(capacity + 1) * 4, md->stream), "tokens clear");
    SMK_HIP(hipMemcpyAsync(md->cos_tab, cos_table, tab, hipMemcpyHostToDevice, md->stream), "cos upload");
    SMK_HIP(hipMemcpyAsync(md->sin_tab, sin_table, tab, hipMemcpyHostToDevice, md->stream), "sin upload");
    md->host_pinned[0] = 0;
    md->host_pinned[1] = 0;
    SMK_HIP(hipMemcpyAsync(md->st, md->host_pinned, sizeof(DecodeState), hipMemcpyHostToDevice, md->stream), "state");
    SMK_HIP(hipStreamSynchronize(md->stream), "reset");
    md->pos = 0;
    if (!md->g_logits) {
        SMK_HIP(allow_lds(attention_for(md->cfg.head_dim), attention_lds(capacity, md->cfg.head_dim)), "attention LDS");
        SMK_HIP(capture(*md, true, &md->g_logits), "capture step");
        SMK_HIP(capture(*md, false, &md->g_plain), "capture step (no logits)");
        SMK_HIP(capture(*md, true, &md->g_next, false), "capture step (embedded by the last argmax)");
    }
    return ok();
}

int smk_llama_step(void* model, int token, float* logits) {
    if (!model) return fail(SMK_ERR_ARGUMENT, "null model");
    auto* md = static_cast<Model*>(model);
    if (!md->capacity) return fail(SMK_ERR_ARGUMENT, "call smk_llama_reset first");
    if (md->pos >= md->capacity)
        return fail(SMK_ERR_ARGUMENT, "KV cache full (" + std::to_string(md->capacity) + " positions)");
    if (token < 0 || token >= md->cfg.vocab) return fail(SMK_ERR_ARGUMENT, "token out of range");
    if (const int rc = use_device()) return rc;
    md->host_pinned[2] = token;
    SMK_HIP(hipMemcpyAsync(md->tokens + md->pos, md->host_pinned + 2, 4, hipMemcpyHostToDevice, md->stream), "token");
    SMK_HIP(hipGraphLaunch(logits ? md->g_logits : md->g_plain, md->stream), "step graph");
    if (logits)
        SMK_HIP(hipMemcpyAsync(logits, md->logits, static_cast<size_t>(md->cfg.vocab) * 4, hipMemcpyDeviceToHost,
                               md->stream),
                "logits download");
    SMK_HIP(hipStreamSynchronize(md->stream), "step");
    ++md->pos;
    return ok();
}

int smk_llama_step_profile(void* model, int token, float* logits, double* section_ms, int n_sections) {
    if (!model || !section_ms) return fail(SMK_ERR_ARGUMENT, "null argument");
    auto* md = static_cast<Model*>(model);
    if (n_sections < kSections) return fail(SMK_ERR_ARGUMENT, "section_ms needs " + std::to_string(kSections) + " entries");
    if (!md->capacity) return fail(SMK_ERR_ARGUMENT, "call smk_llama_reset first");
    if (md->pos >= md->capacity)
        return fail(SMK_ERR_ARGUMENT, "KV cache full (" + std::to_string(md->capacity) + " positions)");
    if (token < 0 || token >= md->cfg.vocab) return fail(SMK_ERR_ARGUMENT, "token out of range");
    if (const int rc = use_device()) return rc;
    md->host_pinned[2] = token;
    SMK_HIP(hipMemcpyAsync(md->tokens + md->pos, md->host_pinned + 2, 4, hipMemcpyHostToDevice, md->stream), "token");
    md->marks.id.clear();
    SMK_HIP(enqueue_step(*md, logits != nullptr, &md->marks), "profiled step");
    SMK_HIP(md->marks.mark(md->stream, kSections), "end mark");
    if (logits)
        SMK_HIP(hipMemcpyAsync(logits, md->logits, static_cast<size_t>(md->cfg.vocab) * 4, hipMemcpyDeviceToHost,
                               md->stream),
                "logits download");
    SMK_HIP(hipStreamSynchronize(md->stream), "step");
    for (size_t i = 0; i + 1 < md->marks.id.size(); ++i) {
        float ms = 0.0f;
        SMK_HIP(hipEventElapsedTime(&ms, md->marks.ev[i], md->marks.ev[i + 1]), "elapsed");
        section_ms[md->marks.id[i]] += ms;
    }
    ++md->pos;
    return ok();
}

int smk_llama_generate(void* model, const int* prompt, int n_prompt, int n_new, int* out, double* seconds) {
    if (!model || !prompt || !out) return fail(SMK_ERR_ARGUMENT, "null argument");
    auto* md = static_cast<Model*>(model);
    if (n_prompt <= 0 || n_new <= 0) return fail(SMK_ERR_ARGUMENT, "n_prompt and n_new must be positive");
    if (md->pos != 0) return fail(SMK_ERR_ARGUMENT, "generate starts from an empty cache: call smk_llama_reset");
    const int steps = n_prompt + n_new - 1;
    if (steps > md->capacity) return fail(SMK_ERR_ARGUMENT, "capacity < n_prompt + n_new - 1");
    for (int i = 0; i < n_prompt; ++i)
        if (prompt[i] < 0 || prompt[i] >= md->cfg.vocab) return fail(SMK_ERR_ARGUMENT, "prompt token out of range");
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipMemcpy(md->tokens, prompt, static_cast<size_t>(n_prompt) * 4, hipMemcpyHostToDevice), "prompt");
    const bool chunked = n_prompt >= 2 && chunked_prefill_ok(*md);
    if (chunked) SMK_HIP(batch_buffers(*md, std::min(md->prefill_rows, n_prompt)), "prompt chunk buffers");
    // Chunked: the last prompt row's argmax runs at position n_prompt - 1.
    md->host_pinned[0] = chunked ? n_prompt - 1 : 0;
    md->host_pinned[1] = n_prompt;
    SMK_HIP(hipMemcpyAsync(md->st, md->host_pinned, sizeof(DecodeState), hipMemcpyHostToDevice, md->stream), "state");
    SMK_HIP(hipEventRecord(md->ev[0], md->stream), "event");
    if (chunked) {
        for (int first = 0; first < n_prompt; first += md->batch_rows) {
            const int P = std::min(md->batch_rows, n_prompt - first);
            SMK_HIP(enqueue_prompt_chunk(*md, first, P, first + P == n_prompt), "prompt chunk");
        }
    } else {
        for (int i = 0; i < n_prompt; ++i) SMK_HIP(hipGraphLaunch(md->g_logits, md->stream), "prefill graph");
    }
    SMK_HIP(hipEventRecord(md->ev[1], md->stream), "event");
    // Every prompt form ends with an argmax, which wrote the first decode step's embedding.
    for (int i = 0; i < n_new - 1; ++i) SMK_HIP(hipGraphLaunch(md->g_next, md->stream), "decode graph");
    SMK_HIP(hipEventRecord(md->ev[2], md->stream), "event");
    SMK_HIP(hipMemcpyAsync(out, md->tokens + n_prompt, static_cast<size_t>(n_new) * 4, hipMemcpyDeviceToHost,
                           md->stream),
            "tokens download");
    SMK_HIP(hipStreamSynchronize(md->stream), "generate");
    md->pos = steps;
    // Back to the step() convention: the given-token count is 0 again.
    md->host_pinned[0] = steps;
    md->host_pinned[1] = 0;
    SMK_HIP(hipMemcpy(md->st, md->host_pinned, sizeof(DecodeState), hipMemcpyHostToDevice), "state");
    if (seconds) {
        float a = 0.0f, b = 0.0f;
        SMK_HIP(hipEventElapsedTime(&a, md->ev[0], md->ev[1]), "elapsed");
        SMK_HIP(hipEventElapsedTime(&b, md->ev[1], md->ev[2]), "elapsed");
        seconds[0] = a * 1e-3;
        seconds[1] = b * 1e-3;
    }
    return ok();
}

int smk_llama_set_prefill_rows(void* model, int rows) {
    if (!model) return fail(SMK_ERR_ARGUMENT, "null model");
    if (rows < 0 || rows > 256) return fail(SMK_ERR_ARGUMENT, "rows must be in [0, 256]");
    static_cast<Model*>(model)->prefill_rows = rows;
    return ok();
}

int smk_llama_info(void* model, int* position, int* capacity, unsigned long long* weight_bytes) {
    if (!model) return fail(SMK_ERR_ARGUMENT, "null model");
    auto* md = static_cast<Model*>(model);
    if (position) *position = md->pos;
    if (capacity) *capacity = md->capacity;
    if (weight_bytes) *weight_bytes = md->weight_bytes;
    return ok();
}

}  // extern "C"
