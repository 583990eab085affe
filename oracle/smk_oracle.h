/*
 * smk_oracle.h -- CPU oracle for the decode-GEMV path.  TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference's scalar semantics
 * (Mattral/simd-ml-kernels 0.3.0, src/kernels/quant/, src/kernels/scalar_kernels.cpp).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
 * and only as the checker: the product (libsmk_hip.so, simd_ml_kernels._core) never
 * links, imports or calls anything under oracle/.
 *
 * How each function is pinned is listed in smk_oracle.c next to it.
 */
#ifndef SMK_ORACLE_H
#define SMK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint16_t smko_fp32_to_fp16(float f);
float smko_fp16_to_fp32(uint16_t h);

int smko_quantize_q8_0_rows(const float* W, int N, int K, uint8_t* out);
int smko_quantize_q4_0_rows(const float* W, int N, int K, uint8_t* out);
int smko_quantize_x_q8(const float* x, int K, int8_t* qs, float* dx);

void smko_gemv_q8_0(int N, int K, const float* x, const uint8_t* Wq, float* y);
void smko_gemv_q4_0(int N, int K, const float* x, const uint8_t* Wq, float* y);

/* Exact per-block int32 sums: out[n*nb + b] = sum_i qw*qx (Q8_0) or sum_i (qw-8)*qx (Q4_0). */
void smko_block_sums_q8_0(int N, int K, const int8_t* qs, const uint8_t* Wq, int32_t* out);
void smko_block_sums_q4_0(int N, int K, const int8_t* qs, const uint8_t* Wq, int32_t* out);

/* C = beta*C + alpha * A * B^T, A [M,lda], B [N,ldb]; elem 0 fp32, 1 fp16, 2 bf16 (bit patterns). */
void smko_gemm_tb(int elem, int M, int N, int K, float alpha, const void* A, int lda, const void* B,
                  int ldb, float beta, float* C, int ldc);

void smko_silu(const float* in, float* out, int n);

/* The reference's SIMD tables' arithmetic orders (AVX2 / AVX-512; see smk_oracle.c). */
void smko_gemv_q4_0_simd(int N, int K, const float* x, const uint8_t* Wq, float* y);
void smko_sgemm_tb_simd(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                        float beta, float* C, int ldc);
void smko_sgemm_nn_simd(int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                        float beta, float* C, int ldc);
float smko_fast_exp(float z);
void smko_silu_simd(const float* in, float* out, int n);
void smko_softmax_simd(const float* in, float* out, int n);

#ifdef __cplusplus
}
#endif
#endif
