/*
 * smk_hip.h -- C ABI of libsmk_hip.so, the MI355X (gfx950) decode-GEMV library.
 *
 * Drop-in boundary for the reference's kernel table (Mattral/simd-ml-kernels 0.3.0,
 * src/dispatch/kernels.hpp:39-78).  Each host-pointer entry point below has the
 * argument list of the KernelTable slot it replaces, plus an int status return:
 * the reference's table functions return void and never fail for data; here a
 * device error (no GPU, out of memory, launch failure) is reported as a status
 * and smk_last_error() holds the message.  Data semantics are unchanged: a
 * non-finite x gives an all-NaN y, K == 0 gives zeros, N == 0 writes nothing.
 *
 * Host-pointer calls copy x in and y out and run on the calling thread's own
 * stream; they return after y is written.  Weights (Wq, B) are uploaded on every
 * call unless their host range was pinned with smk_weights_pin, which keeps one
 * device copy that later calls on any pointer inside that range reuse.
 *
 * smk_d_* entry points take DEVICE pointers and a hipStream_t (as void*; NULL is
 * the null stream), only enqueue work, and never allocate.  Their buffers must
 * be 4-byte aligned; the fast paths also want 16-byte aligned rows.
 *
 * No torch or Python types cross this boundary.
 */
#ifndef SMK_HIP_H
#define SMK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define SMK_OK 0
#define SMK_ERR_ARGUMENT 1      /* invalid shape / pointer / option */
#define SMK_ERR_NO_DEVICE 2     /* no usable gfx950 device */
#define SMK_ERR_DEVICE 3        /* a HIP call failed */
#define SMK_ERR_OUT_OF_MEMORY 4 /* device or pinned allocation failed */
#define SMK_ERR_DATA 5          /* quantizer input not finite, or a block scale overflows float16 */

/* Message of the calling thread's last failure ("" after success). */
const char* smk_last_error(void);
/* Library version string. */
const char* smk_version(void);
/* Device name, arch (e.g. "gfx950"), CU count and HBM bytes of the device in use. */
int smk_device_info(char* name, size_t name_len, char* arch, size_t arch_len, int* compute_units,
                    size_t* hbm_bytes);

/* ─── Host-pointer entry points (KernelTable slots) ───────────────────────── */

/* KernelTable::gemv_q4_0, GemvQ4_0Fn (kernels.hpp:52-53, q4_0.hpp:63-72):
 * y[n] = sum_k x[k] W[n][k], W as N*(K/32) GGUF Q4_0 blocks of 18 bytes, K % 32 == 0. */
int smk_gemv_q4_0(int N, int K, const float* x, const uint8_t* Wq, float* y);
/* KernelTable::gemv_q8_0, GemvQ8_0Fn (kernels.hpp:50-51, q8_0.hpp:18-28, 93-95): 34-byte Q8_0 blocks. */
int smk_gemv_q8_0(int N, int K, const float* x, const uint8_t* Wq, float* y);
/* KernelTable::sgemm, SgemmFn (kernels.hpp:38-41): C = alpha op(A) op(B) + beta C, FP32. */
int smk_sgemm(int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A, int lda, const float* B,
              int ldb, float beta, float* C, int ldc);
/* KernelTable::sgemm_f16, Sgemm16Fn (kernels.hpp:42-45, f16_gemm.hpp:37-44): binary16 A and B,
 * FP32 accumulation and C; trans_b: B stored N x K (x W^T). */
int smk_sgemm_f16(int trans_b, int M, int N, int K, float alpha, const uint16_t* A, int lda, const uint16_t* B,
                  int ldb, float beta, float* C, int ldc);
/* KernelTable::sgemm_bf16, Sgemm16Fn (kernels.hpp:42-45, bf16_gemm.hpp:40-47): BF16 bit patterns. */
int smk_sgemm_bf16(int trans_b, int M, int N, int K, float alpha, const uint16_t* A, int lda, const uint16_t* B,
                   int ldb, float beta, float* C, int ldc);
/* KernelTable::silu, RowFn (kernels.hpp:55, activations.hpp:18-23): out = x / (1 + exp(-x)). */
int smk_silu(const float* in, float* out, int n);
/* KernelTable::softmax_row, RowFn (kernels.hpp:55, activations.hpp:25-28), over `rows` rows of n. */
int smk_softmax(const float* in, float* out, int rows, int n);
/* quantize_q4_0_rows (q4_0.hpp:54-60): W [N, K] -> GGUF Q4_0 blocks; SMK_ERR_DATA on rejection. */
int smk_quantize_q4_0(const float* W, int N, int K, uint8_t* out);
/* quantize_q8_0_rows (q8_0.hpp:53-59): W [N, K] -> GGUF Q8_0 blocks; SMK_ERR_DATA on rejection. */
int smk_quantize_q8_0(const float* W, int N, int K, uint8_t* out);

/* No reference counterpart (the reference computes these in numpy, examples/llama/llama.py:184-187
 * and :169-178 / :387-396): RMSNorm over `rows` rows of n, and RoPE of x [heads, head_dim] with the
 * cos/sin of one position ([head_dim], halves equal); interleaved != 0 rotates pairs (2i, 2i+1). */
int smk_rms_norm(const float* x, const float* weight, float* y, int rows, int n, double eps);
int smk_rope(const float* x, const float* cos, const float* sin, float* y, int heads, int head_dim,
             int interleaved);
/* No reference counterpart (the reference has no batched Q4_0/Q8_0 API, pybind_entry.cpp:956-957):
 * Y [M, N] = X [M, K] W^T, each row of X quantized to Q8 independently (row m equals gemv(X[m])). */
int smk_gemm_q4_0(int M, int N, int K, const float* X, const uint8_t* Wq, float* Y);
int smk_gemm_q8_0(int M, int N, int K, const float* X, const uint8_t* Wq, float* Y);

/* Device-resident weights, keyed by host address range (new: the reference reads host memory). */
int smk_weights_pin(const void* host, size_t nbytes);
int smk_weights_unpin(const void* host);
int smk_weights_stats(size_t* bytes, int* entries);

/* ─── Device-pointer entry points (async on `stream`) ─────────────────────── */
int smk_d_gemv_q4_0(int N, int K, const float* x, const uint8_t* Wq, float* y, void* stream);
int smk_d_gemv_q8_0(int N, int K, const float* x, const uint8_t* Wq, float* y, void* stream);
/* Rows m < M of X [M, ldx] against the same W: Y [M, ldy]; row m of Y equals the one-row call
 * on row m of X bit for bit.  Q4_0 with M >= 2 (K % 64 == 0) runs on the matrix cores, with a
 * scratch buffer the library keeps per (stream, host thread): allocated on the first call of a
 * larger size, which must not be made while the stream is captured into a graph; a buffer it
 * replaces stays allocated until the process ends, so graphs captured earlier stay valid. */
int smk_d_gemm_q4_0(int M, int N, int K, const float* X, int ldx, const uint8_t* Wq, float* Y, int ldy, void* stream);
/* No reference counterpart: for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  smk_d_gemm_q4_0 -- the same
 * kernels, the same bits -- with its scratch in a fixed 4 MiB array of the library (one per GPU,
 * held until the process ends) instead of an allocated buffer; it allocates nothing.  Calls whose
 * x image needs more (about M > 256 rows at K = 14336) are refused with SMK_ERR_ARGUMENT.  All
 * calls on one GPU share the array: calls that overlap on one GPU race (serialize them). */
int smk_d_gemm_q4_0_noalloc(int M, int N, int K, const float* X, int ldx, const uint8_t* Wq, float* Y, int ldy,
                            void* stream);
int smk_d_gemm_q8_0(int M, int N, int K, const float* X, int ldx, const uint8_t* Wq, float* Y, int ldy, void* stream);
/* elem: 0 FP32, 1 FP16, 2 BF16.  C = beta C + alpha A B^T, A [M, lda], B [N, ldb]. */
int smk_d_gemm_tb(int elem, int M, int N, int K, float alpha, const void* A, int lda, const void* B, int ldb,
                  float beta, float* C, int ldc, void* stream);
int smk_d_sgemm(int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A, int lda, const float* B,
                int ldb, float beta, float* C, int ldc, void* stream);
int smk_d_silu(const float* in, float* out, long long n, void* stream);
int smk_d_softmax(const float* in, float* out, int rows, int n, void* stream);
int smk_d_rms_norm(const float* x, const float* weight, float* y, int rows, int n, double eps, void* stream);
int smk_d_rope(const float* x, const float* cos, const float* sin, float* y, int heads, int head_dim, int interleaved,
               void* stream);
/* block_bytes 18 (Q4_0) or 34 (Q8_0).  bad: device int set to 1 on rejection (caller zeroes it). */
int smk_d_quantize(int block_bytes, long long rows, int K, const float* W, uint8_t* out, int* bad, void* stream);
/* Parity helpers: x's Q8 quants/scales (bad as above) and per-block int32 sums [N, K/32]. */
int smk_d_quantize_x_q8(int K, const float* x, int8_t* qs, float* dx, int* bad, void* stream);
int smk_d_block_sums(int block_bytes, int N, int K, const int8_t* qs, const uint8_t* Wq, int32_t* out, void* stream);
/* Self-check of the x quantizer (no reference counterpart): the device's division-free forms of
 * d = amax / 127, id = 1 / d (q8_0_scalar.cpp:52-57) and roundf (:33-40) against IEEE division
 * and the trunc / remainder rounding, over every finite amax >= 0 and every |p| <= 127.5 (about
 * 4.3e9 cases, one synchronous call).  mismatches[0]: scale cases that differ, mismatches[1]:
 * rounding cases that differ; both 0 on a correct device. */
int smk_selfcheck_q8(unsigned* mismatches);
/* HBM read roof: streams nbytes from src (16-byte aligned) with plain or non-temporal 16-byte
 * loads; sink: >= 2048 floats, never read back. */
int smk_d_read_roof(const void* src, size_t nbytes, float* sink, int nontemporal, void* stream);
/* Device-to-device copy of nbytes with a plain 16-byte vector kernel (async on stream); it reads
 * and writes exactly nbytes, which also makes it the calibration kernel of the HBM byte counters. */
int smk_d_copy(void* dst, const void* src, size_t nbytes, void* stream);

/* ─── Device-resident Llama decode ────────────────────────────────────────────
 * No reference counterpart as a library call: the reference runs this loop in numpy around its
 * kernels (examples/llama/llama.py:414-505, step/_attention/generate).  Here the whole step
 * runs on the device from weights uploaded once, with the KV cache in HBM and one HIP graph per
 * token.  Weight types are ggml ids: 0 F32, 2 Q4_0, 8 Q8_0. */
typedef struct smk_llama_config {
    int n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab;
    int matrix_type;      /* type of every layer matrix (q, k, v, o, gate, up, down) */
    int embed_type;       /* type of token_embd */
    int head_type;        /* type of output.weight, or -1: tied to token_embd (llama.py:336-340) */
    int rope_interleaved; /* 1: pairs (2i, 2i+1) (GGUF, llama.py:387-396); 0: halves (llama.py:169-178) */
    double rms_eps;
} smk_llama_config;

/* Tensor ids of smk_llama_set_tensor (GGUF names in comments; layer-wise ids take `layer`). */
#define SMK_LLAMA_TOKEN_EMBD 0  /* token_embd.weight [vocab, hidden] */
#define SMK_LLAMA_OUTPUT_NORM 1 /* output_norm.weight [hidden] F32 */
#define SMK_LLAMA_OUTPUT 2      /* output.weight [vocab, hidden] (only if not tied) */
#define SMK_LLAMA_ATTN_NORM 3   /* blk.L.attn_norm.weight [hidden] F32 */
#define SMK_LLAMA_ATTN_Q 4      /* blk.L.attn_q.weight [n_heads*head_dim, hidden] */
#define SMK_LLAMA_ATTN_K 5      /* blk.L.attn_k.weight [n_kv_heads*head_dim, hidden] */
#define SMK_LLAMA_ATTN_V 6      /* blk.L.attn_v.weight [n_kv_heads*head_dim, hidden] */
#define SMK_LLAMA_ATTN_OUTPUT 7 /* blk.L.attn_output.weight [hidden, n_heads*head_dim] */
#define SMK_LLAMA_FFN_NORM 8    /* blk.L.ffn_norm.weight [hidden] F32 */
#define SMK_LLAMA_FFN_GATE 9    /* blk.L.ffn_gate.weight [ffn, hidden] */
#define SMK_LLAMA_FFN_UP 10     /* blk.L.ffn_up.weight [ffn, hidden] */
#define SMK_LLAMA_FFN_DOWN 11   /* blk.L.ffn_down.weight [hidden, ffn] */

int smk_llama_create(const smk_llama_config* cfg, void** model);
int smk_llama_destroy(void* model);
/* Copy one tensor's bytes (GGUF layout, host memory) into the model; nbytes must match. */
int smk_llama_set_tensor(void* model, int tensor, int layer, const void* host, size_t nbytes);
/* Empty KV cache for `capacity` positions (llama.py:379-385) and the RoPE tables of those
 * positions, cos/sin [capacity, head_dim] as rope_cos_sin makes them (llama.py:162-166). */
int smk_llama_reset(void* model, int capacity, const float* cos_table, const float* sin_table);
/* One token at the next position (llama.py:414-439); logits: host float [vocab], or NULL to skip
 * the lm_head (step(token, logits=False)). */
int smk_llama_step(void* model, int token, float* logits);
/* Greedy decode from an empty cache (llama.py:481-505 with stop_at_eos=False): n_prompt prompt
 * steps, then n_new - 1 decode steps, argmax on the device (np.argmax's first-maximum rule);
 * out: the n_new generated ids; seconds (optional, 2 doubles): prefill and decode time. */
int smk_llama_generate(void* model, const int* prompt, int n_prompt, int n_new, int* out, double* seconds);
int smk_llama_info(void* model, int* position, int* capacity, unsigned long long* weight_bytes);
/* Prompt of smk_llama_generate in chunks of `rows` rows (default 64; 0 or 1: one graph step per
 * prompt token, as the reference's loop, llama.py:491-492).  A chunk runs every matrix product
 * on all its rows at once (Q4_0: the matrix-core kernel); the KV cache and the generated tokens
 * are the same bit for bit either way.  Quantized matrices only (FP32 models run token by token). */
int smk_llama_set_prefill_rows(void* model, int rows);
/* step() run eagerly with a HIP event at every section start (the engine's counterpart of
 * llama.py:441-479, _step_profiled); adds each section's milliseconds into section_ms[0..11):
 * embed, rms_norm, gemv_qkv, rope_kv, attention, gemv_o, gemv_gate_up, silu_mul, gemv_down,
 * lm_head, argmax.  Launch gaps between sections are included. */
int smk_llama_step_profile(void* model, int token, float* logits, double* section_ms, int n_sections);

/* Device memory, copies, streams, events and graphs, for callers without their own runtime
 * objects (the tests and bench.py use these; no other framework is loaded with the library). */
int smk_malloc(void** dptr, size_t nbytes);
int smk_free(void* dptr);
int smk_memcpy_h2d(void* dst, const void* src, size_t nbytes);
int smk_memcpy_d2h(void* dst, const void* src, size_t nbytes);
int smk_memcpy_d2d(void* dst, const void* src, size_t nbytes);
int smk_memset(void* dptr, int byte, size_t nbytes);
int smk_synchronize(void);
int smk_stream_create(void** stream);
int smk_stream_destroy(void* stream);
int smk_stream_synchronize(void* stream);
int smk_event_create(void** event);
int smk_event_destroy(void* event);
int smk_event_record(void* event, void* stream);
int smk_event_elapsed_ms(void* start, void* end, float* ms);
/* Capture the work enqueued on `stream` between begin and end into an executable graph. */
int smk_graph_begin(void* stream);
int smk_graph_end(void* stream, void** graph_exec);
int smk_graph_launch(void* graph_exec, void* stream);
int smk_graph_destroy(void* graph_exec);
/* HIP runtime version in use and the one the library was built against (HIP_VERSION). */
int smk_runtime_version(int* runtime, int* built);

/* Diagnostics: force the quantized GEMV's lanes per row, rows per workgroup, threads per
 * workgroup and per-step row unroll (0 = automatic; the last two apply to one row of x),
 * and report the kernel a call would use ("pairs" or "generic").  Lanes per row 16, 32 or 64
 * and unroll 2 or 4 also set the FP16 / BF16 / FP32 GEMV's (smk_d_gemm_tb, up to 8 rows). */
int smk_set_gemv_tuning(int lanes_per_row, int rows_per_wg, int threads, int unroll);
/* Diagnostics: 1 (default) sums every Q4_0 row in the reference's SIMD order (q4_0_rows.hpp:
 * y bit-exact with its AVX2 / AVX-512 tables); 0 selects the free-order kernel, whose y is
 * within the reference's error bound, for speed comparisons. */
int smk_set_q4_order(int reference_order);
/* Diagnostics: how the reference-order Q4_0 kernel loads one row of x's weights: -1 (default)
 * the built-in choice, 0 each lane its own 36-byte pairs (cached), 1 each wave its rows'
 * contiguous bytes with non-temporal loads staged in LDS, one group of rows ahead, 2 the same two
 * groups ahead (forms 1 and 2 apply where K % 256 == 0, W is 16-byte aligned and a lane takes at
 * most two pairs a row).  y is the same bits in every form.  No reference counterpart: the
 * reference reads its weights from host memory (q4_0_rows.hpp:71-167). */
int smk_set_q4_stream(int mode);
/* Diagnostics: the K-chunk tiled form of the reference-order Q4_0 GEMV for one row of x (tiles of
 * 16 rows x 64 blocks streamed by 576 threads, a wave of its own for the FMA chains): 0 (default)
 * the built-in choice, -1 never (the row-group kernel of smk_set_q4_stream instead), 2, 3 or 4
 * that many tiles in flight wherever the shape allows it (K % 256 == 0, W 16-byte aligned).  y is
 * the same bits either way.  No reference counterpart (its row loop is q4_0_rows.hpp:71-167). */
int smk_set_q4_tiles(int tiles_in_flight);
/* Diagnostics: rows of X from which a Q4_0 product (smk_gemm_q4_0, smk_d_gemm_q4_0) takes the
 * matrix-core kernel (0 = built-in choice; a large value keeps the launches of 8 GEMV rows).
 * No reference counterpart: the reference has no batched Q4_0 product (pybind_entry.cpp:956-957). */
int smk_set_q4_mfma_min_rows(int rows);
const char* smk_gemv_path(int K, const void* Wq);

#ifdef __cplusplus
}
#endif
#endif
