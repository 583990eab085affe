// gemm_q4_mfma.hip -- Q4_0 products Y = X * W^T for several rows of X at once (batched or
// speculative decode, prompt prefill) on gfx950's int8 matrix cores, every row bit-identical
// with the one-row reference-order kernel (q4_0_rows.hpp:71-167).
//
// Why the reference's order survives a matrix core.  Per output, the reference keeps four FP32
// lanes k = 0..3; per block, lane k takes dot_k = the exact integer sum of (q - 8) * qx over
// the eight values {4k..4k+3} and {16+4k..16+4k+3}, and does acc_k = fma(float(dot_k),
// fp16(dw) * dx, acc_k); the output is (acc_0 + acc_2) + (acc_1 + acc_3).  An integer sum is
// the same in any order, so v_mfma_i32_16x16x32_i8 may form the dot_k as long as the four
// lanes' sums stay apart:
//   * the 32 k-slots of one MFMA cover one block, slot 8k + t being value 4k + t (t < 4) or
//     16 + 4k + t - 4 (t >= 4): lane k's eight values, slots 8k..8k+7;
//   * B (32 x 16): column j is row n0 + j of W as signed nibbles q - 8;
//   * A (16 x 32): row 4r + k is x row 4mg + r restricted to lane k -- its quants in slots
//     8k..8k+7 and zeros elsewhere;
//   * D (16 x 16), in the lane that holds D[4r + k][j] for k = 0..3: the four dot_k of x row
//     4mg + r against W row n0 + j.  That lane keeps the reference's four accumulators of that
//     output in registers and applies the block's fma to each, blocks in order.
// Three quarters of A are zeros, so the matrix core does four times the useful integer work;
// the FP32 accumulation (per output and block: four conversions and four fma, as the
// reference) is the real cost at M = 32.
//
// Two launches: quantize_rows_kernel turns the M rows of X into Q8 quants and scales once
// (bit-exact with quantize_x_q8: the same q8_quad), into a scratch buffer laid out as the GEMM's
// LDS image; then the GEMM kernel, each wave owning 16 rows of W for all blocks.
//
// x image (scratch and LDS) of a segment of S = 4 * MG rows of X (the rows of one GEMM
// launch), in chunks of CB blocks, block-major so that every LDS address of a block is a
// compile-time offset:
//   xq [CB][S][32] bytes -- block b of row r at (b S + r) 32, its eight quant dwords in the
//                           order 0 4 1 5 2 6 3 7 (lane k's eight values are the bytes at 8k);
//   dx [CB][S] floats     -- block scales (NaN for a block holding a NaN or an infinity, which
//                           makes its output row NaN, as the reference's rejection);
//   padding of the chunk.  Rows past M hold whatever the buffer held; their products are never
//   stored.
//
// The streaming kernel (K % 1024 == 0, W 16-byte aligned): chunks of 32 blocks.  Per chunk, the
// workgroup loads its 64 rows' 576-byte shares of W with coalesced 16-byte loads and the chunk's
// x image (36 KiB at S = 32), one chunk ahead of the arithmetic; both go through two LDS slots,
// one workgroup barrier per chunk.  Up to four waves share a 16-row tile, each with its own
// groups of x rows (measured on MI355X at 14336 x 4096, M = 32: one wave per tile 65 us, two
// 44 us, four 40 us).  The other
// kernel (K % 64 == 0) holds the whole x image in LDS and reads W straight from memory with
// per-lane 4- and 8-byte slices: correct for every such K, but the scattered slices keep it far
// from the memory roof.
#include "device_common.hpp"
#include "launch.hpp"

#include <algorithm>
#include <map>
#include <thread>
#include <tuple>
#include <vector>
#include <mutex>
#include <utility>

namespace smk {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));

constexpr int kMfmaThreads = 256;           // 4 waves, one 16-row tile of W each
constexpr size_t kMfmaLdsCap = 160 * 1024;  // a gfx950 CU's LDS

// Streaming kernel geometry.
constexpr int kChunkPairs = 16;                                     // pairs of blocks per chunk
constexpr int kChunkBlocks = 2 * kChunkPairs;                       // 32 blocks = 1024 values
constexpr int kWRowBytes = kChunkPairs * 36;                        // a row's share of a chunk
constexpr int kWRowStride = kWRowBytes + 16;                        // in LDS: rows 148 dwords apart
constexpr int kWSlotBytes = 16 * kWRowStride;                       // one wave's 16 rows
constexpr int kWRingBytes = 2 * (kMfmaThreads / kWave) * kWSlotBytes;  // two slots, four waves

// x image chunk bytes (padded to whole 4 KiB rounds of 256 threads x 16 bytes).
__host__ __device__ constexpr int x_chunk_bytes(int S) {
    return (kChunkBlocks * S * 36 + 4095) / 4096 * 4096;
}

struct Layout {
    int rows;            // S: rows of X per launch
    int chunk_blocks;    // CB
    size_t chunk_bytes;  // bytes per chunk of the x image
    size_t dx_off;       // dx offset inside a chunk
    size_t seg_bytes;    // bytes of one segment's x image
    bool streaming;      // the streaming kernel
};

bool streaming_ok(int K, const uint8_t* W) { return K % 1024 == 0 && reinterpret_cast<uintptr_t>(W) % 16 == 0; }

// Whole-image layout (one chunk of all K/32 blocks): bytes of the LDS image.
size_t whole_bytes(int K, int rows) {
    const size_t nb = static_cast<size_t>(K >> 5);
    return (nb * rows * 36 + 1023) & ~static_cast<size_t>(1023);
}

Layout layout(int M, int K, bool streaming) {
    Layout L{};
    int rows = 32;
    if (!streaming)
        while (rows > 4 && whole_bytes(K, rows) > kMfmaLdsCap) rows /= 2;
    while (rows > 4 && rows / 2 >= M) rows /= 2;
    L.rows = rows;
    L.streaming = streaming;
    if (streaming) {
        L.chunk_blocks = kChunkBlocks;
        L.chunk_bytes = x_chunk_bytes(rows);
        L.dx_off = static_cast<size_t>(kChunkBlocks) * rows * 32;
        L.seg_bytes = static_cast<size_t>(K / 1024) * L.chunk_bytes;
    } else {
        if (whole_bytes(K, rows) > kMfmaLdsCap) return Layout{};
        L.chunk_blocks = K >> 5;
        L.chunk_bytes = whole_bytes(K, rows);
        L.dx_off = static_cast<size_t>(K >> 5) * rows * 32;
        L.seg_bytes = L.chunk_bytes;
    }
    return L;
}

// One thread per quad of x (8 consecutive threads per block; K % 32 == 0 keeps a block's quads
// in one 8-lane group).  Threads past the end redo quad 0 and store nothing.
__global__ __launch_bounds__(256) void quantize_rows_kernel(int M, int K, const float* __restrict__ x, int ldx,
                                                            uint8_t* __restrict__ xs, int seg_rows, long long seg_bytes,
                                                            int chunk_blocks, long long chunk_bytes, long long dx_off) {
    const int quads = K >> 2;
    const long long total = static_cast<long long>(M) * quads;
    const long long qd = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    const bool live = qd < total;
    const long long qe = live ? qd : 0;
    const int m = static_cast<int>(qe / quads), kq = static_cast<int>(qe - static_cast<long long>(m) * quads);
    const float* src = x + static_cast<size_t>(m) * ldx + 4 * kq;
    const float v[4] = {src[0], src[1], src[2], src[3]};
    float d;
    int q[4], fin;
    const uint32_t packed = q8_quad(v, d, q, fin);
    const int fin_block = group_sum_int<8>(fin) == 8;
    if (live) {
        const int seg = m / seg_rows, r = m - seg * seg_rows;
        const int b = kq >> 3, k = kq & 7;
        const int c = b / chunk_blocks, bl = b - c * chunk_blocks;
        uint8_t* base = xs + seg * seg_bytes + c * chunk_bytes;
        const int slot = k < 4 ? 2 * k : 2 * (k - 4) + 1;
        const size_t e = static_cast<size_t>(bl) * seg_rows + r;  // (block, row) entry
        reinterpret_cast<uint32_t*>(base + 32 * e)[slot] = packed;
        if (k == 0) reinterpret_cast<float*>(base + dx_off)[e] = fin_block ? d : __builtin_nanf("");
    }
}

// Signed nibbles of one quant dword: low nibbles (values 4k..4k+3) in the low half, high
// nibbles (16+4k..16+4k+3) in the high half, each byte q - 8 (bytes (q | 0x80) - 8 never
// borrow across bytes; xor 0x80 then gives q - 8 in two's complement).
__device__ __forceinline__ long signed_nibbles(uint32_t q) {
    const uint32_t lo = (((q & 0x0f0f0f0fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
    const uint32_t hi = ((((q >> 4) & 0x0f0f0f0fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
    return static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
}

// One pair of blocks (2p, 2p+1) for this lane (W row i = lane % 16, slot group g = lane / 16):
//   w[0], w[1]: pair dwords g, g+1 (block 2p's quant bytes 4g..4g+3 sit 2 bytes into them),
//   w[2]: pair dword 5+g (block 2p+1's quant bytes 4g..4g+3),
//   w[3]: pair dword 0 (block 2p's fp16 scale, low half), w[4]: pair dword 4 (block 2p+1's, high);
//   a: the quants of the A row's x row in this lane's slot group; dx: the block scales of D's
//   x row.
template <int MG>
struct PairOps {
    uint32_t w[5];
    long a[2][MG];
    float dx[2][MG];
};

// x operands of blocks 2p, 2p+1 of an x image chunk (S rows per block), MG groups of 4 rows.
template <int MG, int S = 4 * MG>
__device__ __forceinline__ void read_x(const uint8_t* __restrict__ xq_lane, const float* __restrict__ dx_lane, int p,
                                       PairOps<MG>& o) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int b = 2 * p + h;
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) {
            o.a[h][mg] = *reinterpret_cast<const long*>(xq_lane + (b * S + 4 * mg) * 32);
            o.dx[h][mg] = dx_lane[b * S + 4 * mg];
        }
    }
}

// Both blocks of a pair: per block, MG products and the reference's four fma per output.
// on: this lane's A slots belong to its A row's lane k (the other three quarters are zero).
template <int MG>
__device__ __forceinline__ void mfma_pair(const PairOps<MG>& o, bool on, float (&acc)[MG][4]) {
    const i32x4 zero = {0, 0, 0, 0};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const long bw = signed_nibbles(h == 0 ? skip2(o.w[1], o.w[0]) : o.w[2]);
        const float dw = half_bits_to_float(h == 0 ? o.w[3] : o.w[4] >> 16);
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) {
            const i32x4 dk = __builtin_amdgcn_mfma_i32_16x16x32_i8(on ? o.a[h][mg] : 0L, bw, zero, 0, 0, 0);
            const float s = dw * o.dx[h][mg];
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[mg][k] = fmaf(static_cast<float>(dk[k]), s, acc[mg][k]);
        }
    }
}

template <int MG>
__device__ __forceinline__ void store_rows(const float (&acc)[MG][4], int M, int N, int n, int g, float* __restrict__ y,
                                           int ldy, int accumulate) {
    if (n >= N) return;
#pragma unroll
    for (int mg = 0; mg < MG; ++mg) {
        const int m = 4 * mg + g;
        if (m < M) {
            const float v = (acc[mg][0] + acc[mg][2]) + (acc[mg][1] + acc[mg][3]);
            float* yp = y + static_cast<size_t>(m) * ldy + n;
            *yp = accumulate ? *yp + v : v;
        }
    }
}

// ─── streaming kernel ────────────────────────────────────────────────────────

// LDS: two x slots of x_chunk_bytes(S), then (at w_ring = their size) two W slots of four tiles.
// Rows m < M (M <= 4 MG) of one segment against W rows [64 blockIdx, 64 blockIdx + 64): four
// 16-row tiles, SPLIT waves per tile (wave w: tile w % 4, x row groups [(w / 4) MG / SPLIT,
// (w / 4 + 1) MG / SPLIT)), so that several waves per SIMD hide each other's latencies when M
// allows.  With few rows of W (fewer workgroups than CUs) the grid's y dimension splits the x
// row groups further: workgroup (t, u) takes groups [u MG / YS, (u + 1) MG / YS) of W rows
// [64 t, 64 t + 64), reading those rows of W once per u (from the caches after the first).
// K % 1024 == 0, W 16-byte aligned, N even.  Waves past N run on clamped rows and store nothing
// (every wave reaches every barrier).
template <int MG, int SPLIT, int YS>
__global__ __launch_bounds__(kMfmaThreads * SPLIT) void gemm_q4_mfma_kernel(int M, int N, int K,
                                                                            const uint8_t* __restrict__ seg,
                                                                            const uint8_t* __restrict__ W,
                                                                            float* __restrict__ y, int ldy,
                                                                            int accumulate, int w_ring) {
    constexpr int S = 4 * MG, MGW = MG / (SPLIT * YS), NT = kMfmaThreads * SPLIT;
    static_assert(MGW * SPLIT * YS == MG, "x row groups split evenly over waves and grid rows");
    constexpr int XC = x_chunk_bytes(S);
    constexpr int XPC = XC / 16;                        // 16-byte pieces of an x chunk
    constexpr int WPC = 4 * 16 * kWRowBytes / 16;       // 16-byte pieces of a W chunk (4 tiles)
    constexpr int XP = (XPC + NT - 1) / NT, WP = (WPC + NT - 1) / NT;
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int tile = wave & 3, mg0 = (static_cast<int>(blockIdx.y) * SPLIT + (wave >> 2)) * MGW;
    const int nb = K >> 5, nch = nb / kChunkBlocks;
    const size_t row_bytes = static_cast<size_t>(nb) * 18;
    const int nw = blockIdx.x * 64;                     // first W row of the workgroup
    const int g = lane >> 4, i = lane & 15;

    // Chunk c into registers: W piece q = (tile, row, 16-byte column) of 4 x 16 rows x 36.
    auto load_chunk = [&](int c, u32x4(&wr)[WP], u32x4(&xr)[XP]) {
#pragma unroll
        for (int j = 0; j < WP; ++j) {
            const int q = j * NT + tid;
            if (WPC % NT == 0 || q < WPC) {
                const int r = q / 36, col = q - 36 * r;   // r: row of the workgroup's 64
                const int row = min(nw + r, N - 1);
                wr[j] = *reinterpret_cast<const u32x4*>(W + row * row_bytes + static_cast<size_t>(c) * kWRowBytes +
                                                        16 * col);
            }
        }
        const u32x4* xs = reinterpret_cast<const u32x4*>(seg + static_cast<size_t>(c) * XC);
#pragma unroll
        for (int j = 0; j < XP; ++j) {
            const int q = j * NT + tid;
            if (XPC % NT == 0 || q < XPC) xr[j] = xs[q];
        }
    };
    auto store_chunk = [&](int slot, const u32x4(&wr)[WP], const u32x4(&xr)[XP]) {
        uint8_t* wdst = lds + w_ring + slot * (kWRingBytes / 2);
#pragma unroll
        for (int j = 0; j < WP; ++j) {
            const int q = j * NT + tid;
            if (WPC % NT == 0 || q < WPC) {
                const int r = q / 36, col = q - 36 * r;   // tile r / 16, row r % 16 of it
                *reinterpret_cast<u32x4*>(wdst + (r >> 4) * kWSlotBytes + (r & 15) * kWRowStride + 16 * col) = wr[j];
            }
        }
        u32x4* xdst = reinterpret_cast<u32x4*>(lds + slot * XC);
#pragma unroll
        for (int j = 0; j < XP; ++j) {
            const int q = j * NT + tid;
            if (XPC % NT == 0 || q < XPC) xdst[q] = xr[j];
        }
    };

    const bool on = g == (i & 3);
    float acc[MGW][4];
#pragma unroll
    for (int mg = 0; mg < MGW; ++mg)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[mg][k] = 0.0f;

    auto compute_chunk = [&](int slot) {
        // Every LDS read of a chunk is a per-lane base plus an offset below 64 KiB (the LDS
        // instructions' immediate): the x ring comes first, and the W ring's offset (2 XC) is a
        // kernel argument, so that the compiler cannot fold it into the immediates.
        const uint8_t* wrow = lds + w_ring + slot * (kWRingBytes / 2) + tile * kWSlotBytes + i * kWRowStride;
        const uint8_t* xsl = lds + slot * XC;
        const uint8_t* xq_lane = xsl + (4 * mg0 + (i >> 2)) * 32 + 8 * g;
        const float* dx_lane = reinterpret_cast<const float*>(xsl + kChunkBlocks * S * 32) + 4 * mg0 + g;
        auto read_ops = [&](int p, PairOps<MGW>& o) {
            const uint8_t* wp = wrow + 36 * p;
            o.w[0] = *reinterpret_cast<const uint32_t*>(wp + 4 * g);
            o.w[1] = *reinterpret_cast<const uint32_t*>(wp + 4 * g + 4);
            o.w[2] = *reinterpret_cast<const uint32_t*>(wp + 20 + 4 * g);
            o.w[3] = *reinterpret_cast<const uint32_t*>(wp);
            o.w[4] = *reinterpret_cast<const uint32_t*>(wp + 16);
            read_x<MGW, S>(xq_lane, dx_lane, p, o);
        };
        PairOps<MGW> cur;
        read_ops(0, cur);
#pragma unroll 2
        for (int u = 0; u < kChunkPairs; ++u) {
            PairOps<MGW> nxt;
            read_ops(u + 1 < kChunkPairs ? u + 1 : u, nxt);
            mfma_pair<MGW>(cur, on, acc);
            cur = nxt;
        }
    };

    // One chunk in flight: chunk c + 1's loads run during chunk c's arithmetic.  (Two chunks in
    // flight, in two register sets, measured slower on MI355X at M <= 4.)
    u32x4 wr[WP], xr[XP];
    load_chunk(0, wr, xr);
    store_chunk(0, wr, xr);
    if (nch > 1) load_chunk(1, wr, xr);
    lds_barrier();
    for (int c = 0; c < nch; ++c) {
        compute_chunk(c & 1);
        if (c + 1 < nch) store_chunk((c & 1) ^ 1, wr, xr);
        if (c + 2 < nch) load_chunk(c + 2, wr, xr);
        lds_barrier();
    }
    store_rows<MGW>(acc, M - 4 * mg0, N, nw + 16 * tile + i, g, y + static_cast<size_t>(4 * mg0) * ldy, ldy,
                    accumulate);
}

// ─── whole-image kernel (any K % 64 == 0) ────────────────────────────────────

// Per lane and pair p of its W row: the five dwords of PairOps::w.
__device__ __forceinline__ void load_pair_slices(const uint8_t* __restrict__ wrow, int p, int g, uint32_t (&r)[5]) {
    const uint32_t* P = reinterpret_cast<const uint32_t*>(wrow + 36 * static_cast<size_t>(p));
    const u32x2a4 a = *reinterpret_cast<const u32x2a4*>(P + g);
    r[0] = a.x;
    r[1] = a.y;
    r[2] = P[5 + g];
    r[3] = P[0];
    r[4] = P[4];
}

// The whole x image in LDS (global_load_lds), W slices straight from memory PD pairs ahead.
// K % 64 == 0, W 4-byte aligned, N even.
template <int MG, int PD>
__global__ __launch_bounds__(kMfmaThreads) void gemm_q4_mfma_whole_kernel(int M, int N, int K,
                                                                          const uint8_t* __restrict__ seg,
                                                                          int seg_bytes, int dx_off,
                                                                          const uint8_t* __restrict__ W,
                                                                          float* __restrict__ y, int ldy,
                                                                          int accumulate) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int nb = K >> 5, pairs = nb >> 1;
    const int n0 = (blockIdx.x * (kMfmaThreads / kWave) + wave) * 16;
    const int g = lane >> 4, i = lane & 15;
    const int row = min(n0 + i, N - 1);
    const uint8_t* wrow = W + static_cast<size_t>(row) * nb * 18;

    // The segment's image into LDS, every wave a share of 1 KiB rounds, then the first PD pairs
    // of weights; one wait covers both (the weights are needed first anyway).
    {
        const u32x4* src = reinterpret_cast<const u32x4*>(seg);
        u32x4* dst = reinterpret_cast<u32x4*>(lds);
        const int n16 = seg_bytes >> 4;
        for (int base = wave * kWave; base < n16; base += kMfmaThreads)
            __builtin_amdgcn_global_load_lds(src + base + lane, dst + base, 16, 0, 0);
    }
    uint32_t w[PD][5];
#pragma unroll
    for (int u = 0; u < PD; ++u) load_pair_slices(wrow, u < pairs ? u : pairs - 1, g, w[u]);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the LDS image has landed
    lds_barrier();

    // This lane's A entries: x row 4 mg + (i >> 2), slot group g; its D entries: x row 4 mg + g.
    const uint8_t* xq_lane = lds + (i >> 2) * 32 + 8 * g;
    const float* dx_lane = reinterpret_cast<const float*>(lds + dx_off) + g;
    const bool on = g == (i & 3);

    float acc[MG][4];
#pragma unroll
    for (int mg = 0; mg < MG; ++mg)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[mg][k] = 0.0f;

    PairOps<MG> xc;
    read_x<MG>(xq_lane, dx_lane, 0, xc);
    int p0 = 0;
    for (; p0 + PD <= pairs; p0 += PD) {
#pragma unroll
        for (int u = 0; u < PD; ++u) {
            PairOps<MG> xn;
            const int pn = p0 + u + 1;
            read_x<MG>(xq_lane, dx_lane, pn < pairs ? pn : pairs - 1, xn);
#pragma unroll
            for (int t = 0; t < 5; ++t) xc.w[t] = w[u][t];
            mfma_pair<MG>(xc, on, acc);
            const int pw = p0 + u + PD;
            load_pair_slices(wrow, pw < pairs ? pw : pairs - 1, g, w[u]);
            xc = xn;
            __builtin_amdgcn_sched_barrier(0);  // keep each pair's work in place (register pressure)
        }
    }
#pragma unroll
    for (int u = 0; u < PD; ++u) {
        if (p0 + u < pairs) {
            PairOps<MG> xn;
            const int pn = p0 + u + 1;
            read_x<MG>(xq_lane, dx_lane, pn < pairs ? pn : pairs - 1, xn);
#pragma unroll
            for (int t = 0; t < 5; ++t) xc.w[t] = w[u][t];
            mfma_pair<MG>(xc, on, acc);
            xc = xn;
        }
    }
    store_rows<MG>(acc, M, N, n0 + i, g, y, ldy, accumulate);
}

template <int MG, int SPLIT, int YS>
hipError_t launch_streaming(int M, int N, int K, const uint8_t* seg, const uint8_t* W, float* y, int ldy, int acc,
                            hipStream_t stream) {
    auto kernel = gemm_q4_mfma_kernel<MG, SPLIT, YS>;
    const size_t lds = kWRingBytes + 2 * static_cast<size_t>(x_chunk_bytes(4 * MG));
    if (const hipError_t e = allow_lds(kernel, lds); e != hipSuccess) return e;
    const int grid = (N + 63) / 64;
    const int w_ring = 2 * x_chunk_bytes(4 * MG);  // the W ring follows the two x slots
    hipLaunchKernelGGL(kernel, dim3(grid, YS), dim3(kMfmaThreads * SPLIT), lds, stream, M, N, K, seg, W, y, ldy, acc,
                       w_ring);
    return hipGetLastError();
}

template <int MG, int PD>
hipError_t launch_whole(int M, int N, int K, const uint8_t* seg, const Layout& L, const uint8_t* W, float* y, int ldy,
                        int acc, hipStream_t stream) {
    auto kernel = gemm_q4_mfma_whole_kernel<MG, PD>;
    if (const hipError_t e = allow_lds(kernel, L.seg_bytes); e != hipSuccess) return e;
    const int grid = ((N + 15) / 16 + 3) / 4;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kMfmaThreads), L.seg_bytes, stream, M, N, K, seg,
                       static_cast<int>(L.seg_bytes), static_cast<int>(L.dx_off), W, y, ldy, acc);
    return hipGetLastError();
}

}  // namespace

bool gemm_q4_mfma_ok(int M, int N, int K, const uint8_t* W) {
    return M >= 1 && N >= 2 && (N & 1) == 0 && K >= 64 && K % 64 == 0 &&
           reinterpret_cast<uintptr_t>(W) % 4 == 0 && layout(M, K, streaming_ok(K, W)).rows > 0;
}

size_t gemm_q4_mfma_workspace(int M, int K) {
    // The larger of the two layouts (the kernel is chosen by W's alignment at the call).
    size_t best = 0;
    for (const bool s : {true, false}) {
        if (s && K % 1024) continue;
        const Layout L = layout(M, K, s);
        if (L.rows > 0) best = std::max(best, static_cast<size_t>((M + L.rows - 1) / L.rows) * L.seg_bytes);
    }
    return best;
}

// Scratch of the batched path, one buffer per (device, stream, host thread): launches on one
// stream from one thread run in order, so a buffer is never used by two products at once, and
// two threads sharing a stream (the null stream, say) get buffers of their own.  A buffer only
// grows, outside stream capture; the buffer it replaces is never freed (a graph captured earlier
// on that stream holds its address in its nodes and may be replayed later), so every buffer this
// function hands out stays valid until the process ends.
hipError_t stream_workspace(hipStream_t stream, size_t bytes, void** out) {
    struct Slot {
        void* p = nullptr;
        size_t cap = 0;
    };
    static std::mutex mu;
    static std::map<std::tuple<int, hipStream_t, std::thread::id>, Slot> cache;
    static std::vector<void*> retired;  // superseded buffers, kept alive for captured graphs
    int dev = 0;
    if (const hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(mu);
    Slot& slot = cache[{dev, stream, std::this_thread::get_id()}];
    if (slot.cap < bytes) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        if (const hipError_t e = hipStreamIsCapturing(stream, &st); e != hipSuccess) return e;
        if (st != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
        const size_t grown = std::max(bytes, static_cast<size_t>(1) << 20);
        void* p = nullptr;
        if (const hipError_t e = hipMalloc(&p, grown); e != hipSuccess) return e;
        if (slot.p) retired.push_back(slot.p);
        slot.p = p;
        slot.cap = grown;
    }
    *out = slot.p;
    return hipSuccess;
}

hipError_t gemm_q4_mfma(int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y, int ldy, int acc,
                        void* workspace, hipStream_t stream) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (!gemm_q4_mfma_ok(M, N, K, W) || !workspace) return hipErrorInvalidValue;
    const Layout L = layout(M, K, streaming_ok(K, W));
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    {
        const long long quads = static_cast<long long>(M) * (K >> 2);
        const int grid = static_cast<int>((quads + 255) / 256);
        hipLaunchKernelGGL(quantize_rows_kernel, dim3(grid), dim3(256), 0, stream, M, K, x, ldx, ws, L.rows,
                           static_cast<long long>(L.seg_bytes), L.chunk_blocks, static_cast<long long>(L.chunk_bytes),
                           static_cast<long long>(L.dx_off));
        if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    // Grid rows of the streaming kernel: split the x row groups while the workgroups of 64 W rows
    // leave CUs idle (at most 256 workgroups; one group of 4 x rows per wave at the finest).
    int ys = 1;
    {
        const int gx = (N + 63) / 64;
        while (2 * ys <= L.rows / 4 && 2 * ys <= 8 && gx * 2 * ys <= 256) ys *= 2;
    }
    for (int m0 = 0; m0 < M; m0 += L.rows) {
        const int mr = std::min(L.rows, M - m0);
        const uint8_t* seg = ws + static_cast<size_t>(m0 / L.rows) * L.seg_bytes;
        float* ym = y + static_cast<size_t>(m0) * ldy;
        hipError_t e;
        if (L.streaming) {
            switch (L.rows) {
                case 4: e = launch_streaming<1, 1, 1>(mr, N, K, seg, W, ym, ldy, acc, stream); break;
                case 8: e = ys == 1 ? launch_streaming<2, 2, 1>(mr, N, K, seg, W, ym, ldy, acc, stream)
                                    : launch_streaming<2, 1, 2>(mr, N, K, seg, W, ym, ldy, acc, stream);
                    break;
                case 16:
                    e = ys == 1   ? launch_streaming<4, 4, 1>(mr, N, K, seg, W, ym, ldy, acc, stream)
                        : ys == 2 ? launch_streaming<4, 2, 2>(mr, N, K, seg, W, ym, ldy, acc, stream)
                                  : launch_streaming<4, 1, 4>(mr, N, K, seg, W, ym, ldy, acc, stream);
                    break;
                default:
                    e = ys == 1   ? launch_streaming<8, 4, 1>(mr, N, K, seg, W, ym, ldy, acc, stream)
                        : ys == 2 ? launch_streaming<8, 4, 2>(mr, N, K, seg, W, ym, ldy, acc, stream)
                        : ys == 4 ? launch_streaming<8, 2, 4>(mr, N, K, seg, W, ym, ldy, acc, stream)
                                  : launch_streaming<8, 1, 8>(mr, N, K, seg, W, ym, ldy, acc, stream);
                    break;
            }
        } else {
            switch (L.rows) {
                case 4: e = launch_whole<1, 8>(mr, N, K, seg, L, W, ym, ldy, acc, stream); break;
                case 8: e = launch_whole<2, 8>(mr, N, K, seg, L, W, ym, ldy, acc, stream); break;
                case 16: e = launch_whole<4, 4>(mr, N, K, seg, L, W, ym, ldy, acc, stream); break;
                default: e = launch_whole<8, 4>(mr, N, K, seg, L, W, ym, ldy, acc, stream); break;
            }
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace smk
