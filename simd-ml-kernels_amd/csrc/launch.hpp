// launch.hpp -- internal launchers of the gfx950 kernels (device pointers, async on a stream).
// The C ABI (smk_hip.h) is built on these; nothing here is exported.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace smk {

// Block bytes of the two GGUF weight formats.
constexpr int kQ4_0Bytes = 18;
constexpr int kQ8_0Bytes = 34;

// Options of the quantized GEMV; zero fields take the built-in choice.
struct GemvTuning {
    int lanes_per_row = 0;  // 8, 16, 32 or 64 lanes share one row of W
    int rows_per_wg = 0;    // rows of W per workgroup
    int threads = 0;        // threads per workgroup: 256, 512 or 1024 (one row of x only)
    int unroll = 0;         // rows per lane group per step: 1, 2 or 4 (one row of x only)
    int accumulate = 0;     // 1: y = y + x.W^T (one float32 add per output: a residual update)
    int unordered = 0;      // Q4_0 only, diagnostics: the free-order pair kernel instead of the
                            // reference's SIMD summation order
    const float* norm_w = nullptr;  // Q4_0, one row of x: use RMSNorm(x) * norm_w instead of x
    double norm_eps = 0.0;          // (numpy-exact, as rms_norm), K <= 8192, N even
    int silu_pairs = 0;             // Q4_0, one row of x, N even: rows 2n, 2n+1 are (gate, up);
                                    // y[n] = silu(gate) * up (y has N / 2 entries)
    int mfma_min_rows = 0;          // Q4_0 in the reference order: rows of x from which the
                                    // matrix-core kernel takes the product (0: built-in choice)
    int stream_weights = 0;         // Q4_0, one row of x: 1 streams the weights with
                                    // non-temporal loads wherever the shape allows (a decode
                                    // step: the caches keep its activations and KV cache)
    void* workspace = nullptr;      // scratch of the batched Q4_0 path supplied by the caller
    size_t workspace_bytes = 0;     // (instead of the stream's buffer): its size in bytes
};

// y[m*ldy + n] = sum_k x[m*ldx + k] * W[n][k] for m < M, W in GGUF Q4_0 (block_bytes 18) or
// Q8_0 (34) blocks; each row of x is quantized to Q8 blocks (inside the GEMV kernel, or once
// by the batched Q4_0 path's quantizer).  A row of x with a NaN or +-Inf makes its whole row
// of y NaN; K == 0 gives zeros.  K % 32 == 0.  Several rows of x against Q4_0 take the matrix-core
// kernel (gemm_q4_mfma) when its shape conditions hold, with the stream's scratch buffer
// (stream_workspace); otherwise launches of at most 8 rows.
hipError_t gemv_quant(int block_bytes, int M, int N, int K, const float* x, int ldx, const uint8_t* W,
                      float* y, int ldy, hipStream_t stream, const GemvTuning* tuning = nullptr);

// The batched Q4_0 product on the matrix cores, every row bit-identical with the one-row
// reference-order kernel: M >= 1 rows of x, N even, K % 64 == 0, W 4-byte aligned
// (gemm_q4_mfma_ok).  workspace: gemm_q4_mfma_workspace(M, K) bytes of device memory, 16-byte
// aligned, used by the launches on `stream` only.  acc: y = y + x.W^T.
bool gemm_q4_mfma_ok(int M, int N, int K, const uint8_t* W);
size_t gemm_q4_mfma_workspace(int M, int K);
hipError_t gemm_q4_mfma(int M, int N, int K, const float* x, int ldx, const uint8_t* W, float* y, int ldy, int acc,
                        void* workspace, hipStream_t stream);
// A scratch buffer of at least `bytes` owned by the library for launches on `stream` of the
// current device (grown outside graph capture only: the first call of a size must not be
// captured).
hipError_t stream_workspace(hipStream_t stream, size_t bytes, void** out);

// Compute units of the device (workgroup counts of the GEMV follow it).
void set_compute_units(int cus);

// Diagnostics: the weight-load form of the reference-order Q4_0 kernel for one row of x (-1 the
// built-in choice, 0 pair loads, 1 streamed one group ahead, 2 two groups ahead; a form applies
// where the shape allows it).  Not synchronised with launches in flight.
void set_q4_stream(int mode);

// Diagnostics: the K-chunk tiled kernel of the reference-order Q4_0 GEMV for one row of x (0 the
// built-in choice, -1 never, 2..4 that many tiles in flight wherever the shape allows it).  Not
// synchronised with launches in flight.
void set_q4_tiles(int tiles);

// Diagnostics: lanes per row (16, 32 or 64; 0 automatic) and rows per lane group (2 or 4) of
// the FP16 / BF16 / FP32 GEMV.
void set_lowp_tuning(int lanes_per_row, int unroll);

// The kernel gemv_quant would launch, for reports: "pairs" or "generic".
const char* gemv_quant_path(int block_bytes, int N, int K, const uint8_t* W);

// x -> Q8 quants and FP32 scales on the device (qs int8 [K], dx float [K/32]); *bad = 1 when x
// holds a NaN or +-Inf.  Bit-exact with the reference's quantize_x_q8.
hipError_t quantize_x_q8(int K, const float* x, int8_t* qs, float* dx, int* bad, hipStream_t stream);

// Exhaustive device check of the x quantizer's division-free scale and rounding against the IEEE
// forms: counts[0] += scale mismatches, counts[1] += rounding mismatches (counts zeroed by the
// caller; 0 and 0 expected).
hipError_t q8_selfcheck(unsigned* counts, hipStream_t stream);

// Per-block int32 sums of x's Q8 quants against W's blocks: out [N, K/32].
hipError_t block_sums(int block_bytes, int N, int K, const int8_t* qs, const uint8_t* W, int32_t* out,
                      hipStream_t stream);

// W float [rows, K] -> GGUF blocks (block_bytes 18 or 34) bit-exact with ggml's reference
// quantizers; *bad = 1 if W holds a NaN/Inf or a block scale overflows float16.
hipError_t quantize_weights(int block_bytes, long long rows, int K, const float* W, uint8_t* out, int* bad,
                            hipStream_t stream);

// C = beta*C + alpha * A * B^T with A [M, lda] and B [N, ldb] of element type elem (0 fp32,
// 1 fp16, 2 bf16), FP32 accumulation.  M <= 8 takes the row-streaming GEMV kernel.
hipError_t gemm_tb(int elem, int M, int N, int K, float alpha, const void* A, int lda, const void* B, int ldb,
                   float beta, float* C, int ldc, hipStream_t stream);

// C = beta*C + alpha * op(A) * op(B), FP32, any transposes (small operands; attention helper).
hipError_t sgemm_generic(bool trans_a, bool trans_b, int M, int N, int K, float alpha, const float* A, int lda,
                         const float* B, int ldb, float beta, float* C, int ldc, hipStream_t stream);

hipError_t silu(const float* in, float* out, long long n, hipStream_t stream);
hipError_t softmax_rows(const float* in, float* out, int rows, int n, hipStream_t stream);
hipError_t rms_norm(const float* x, const float* w, float* y, int rows, int n, double eps, hipStream_t stream);
hipError_t rope(const float* x, const float* cos, const float* sin, float* y, int heads, int head_dim,
                bool interleaved, hipStream_t stream);
hipError_t fill(float* y, long long n, float value, hipStream_t stream);

// Streams `bytes` of src (16-byte aligned) with plain or non-temporal 16-byte loads and writes
// nothing (unless an improbable xor matches): the HBM read roof.
hipError_t read_roof(const void* src, size_t bytes, float* sink, bool nontemporal, hipStream_t stream);
// Device-to-device copy with a plain vector kernel (hipMemcpyAsync when a pointer is not
// 16-byte aligned).
hipError_t copy_bytes(void* dst, const void* src, size_t bytes, hipStream_t stream);

}  // namespace smk
