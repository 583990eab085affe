// ref_shim.cpp -- C entry points over the REFERENCE's own kernel tables.  TEST
// INFRASTRUCTURE ONLY.
//
// oracle/Makefile compiles the reference's kernel units where they lie
// (/root/reference/src, never copied) together with this file into
// oracle/_ref/libsmk_ref.so.  Tests use it to pin the oracle restatement to the
// real reference (bit-exact quantizers, bit-exact scalar-table GEMV), and
// bench.py's cpu_baseline leg times the reference's best SIMD path with it.
// The product never loads it.
#include "dispatch/kernels.hpp"
#include "kernels/gemm/avx2_gemm_packed.hpp"
#include "kernels/quant/q4_0.hpp"
#include "kernels/quant/q8_0.hpp"

#include <cstdint>

namespace {
const simd_ml::KernelTable* table(int isa) {
    if (isa < 0 || isa >= simd_ml::kNumIsa) return nullptr;
    return simd_ml::kernels_for(static_cast<simd_ml::Isa>(isa));
}
}  // namespace

extern "C" {

// 1 if the reference's table for isa (0 scalar, 1 avx2, 2 avx512) runs on this CPU.
int ref_table_available(int isa) { return table(isa) != nullptr; }

const char* ref_table_flags(int isa) {
    const simd_ml::KernelTable* t = table(isa);
    return t ? t->flags : "";
}

// Inner loop gemv_q8_0 / gemv_q4_0 of the given table would use ("avx512_vnni", ...).
const char* ref_q8_0_path(int isa) {
    const simd_ml::KernelTable* t = table(isa);
    if (!t) return "";
    const simd_ml::KernelTable& keep = simd_ml::kernels();
    simd_ml::use_kernels(static_cast<simd_ml::Isa>(isa));
    const char* p = simd_ml::quant::q8_0_path();
    simd_ml::use_kernels(keep.isa);
    return p;
}

int ref_gemv_q4_0(int isa, int N, int K, const float* x, const uint8_t* Wq, float* y) {
    const simd_ml::KernelTable* t = table(isa);
    if (!t) return -1;
    t->gemv_q4_0(N, K, x, Wq, y);
    return 0;
}

int ref_gemv_q8_0(int isa, int N, int K, const float* x, const uint8_t* Wq, float* y) {
    const simd_ml::KernelTable* t = table(isa);
    if (!t) return -1;
    t->gemv_q8_0(N, K, x, Wq, y);
    return 0;
}

int ref_sgemm(int isa, int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A, int lda,
              const float* B, int ldb, float beta, float* C, int ldc) {
    const simd_ml::KernelTable* t = table(isa);
    if (!t) return -1;
    t->sgemm(trans_a != 0, trans_b != 0, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    return 0;
}

int ref_sgemm_f16(int isa, int trans_b, int M, int N, int K, float alpha, const uint16_t* A, int lda,
                  const uint16_t* B, int ldb, float beta, float* C, int ldc) {
    const simd_ml::KernelTable* t = table(isa);
    if (!t) return -1;
    t->sgemm_f16(trans_b != 0, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    return 0;
}

int ref_sgemm_bf16(int isa, int trans_b, int M, int N, int K, float alpha, const uint16_t* A, int lda,
                   const uint16_t* B, int ldb, float beta, float* C, int ldc) {
    const simd_ml::KernelTable* t = table(isa);
    if (!t) return -1;
    t->sgemm_bf16(trans_b != 0, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    return 0;
}

int ref_silu(int isa, const float* in, float* out, int n) {
    const simd_ml::KernelTable* t = table(isa);
    if (!t) return -1;
    t->silu(in, out, n);
    return 0;
}

int ref_softmax_row(int isa, const float* in, float* out, int n) {
    const simd_ml::KernelTable* t = table(isa);
    if (!t) return -1;
    t->softmax_row(in, out, n);
    return 0;
}

int ref_quantize_q4_0(const float* W, int N, int K, uint8_t* out) {
    return simd_ml::quant::quantize_q4_0_rows(W, N, K, out) ? 1 : 0;
}

int ref_quantize_q8_0(const float* W, int N, int K, uint8_t* out) {
    return simd_ml::quant::quantize_q8_0_rows(W, N, K, out) ? 1 : 0;
}

int ref_quantize_x_q8(const float* x, int K, int8_t* qs, float* dx) {
    return simd_ml::quant::quantize_x_q8(x, K, qs, dx) ? 1 : 0;
}

uint16_t ref_fp32_to_fp16(float f) { return simd_ml::quant::fp32_to_fp16(f); }
float ref_fp16_to_fp32(uint16_t h) { return simd_ml::quant::fp16_to_fp32(h); }

void ref_set_num_threads(int n) { simd_ml::gemm::set_num_threads(n); }
int ref_get_num_threads(void) { return simd_ml::gemm::get_num_threads(); }

}  // extern "C"
