// kernel_table.hpp -- the host side of the plugin boundary: one KernelTable, "gfx950", whose
// slots have the reference's function-pointer signatures (src/dispatch/kernels.hpp:38-78) and
// run on the MI355X through the C ABI of libsmk_hip.so (include/smk_hip.h).
//
// The reference's table functions return void and never fail for data.  A device failure
// here (no GPU, out of memory, launch error) throws DeviceError, which the bindings turn into
// RuntimeError.  There is no CPU table and no CPU fallback: without a gfx950 device every
// slot throws.
#pragma once

#include "smk_hip.h"

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace smk_host {

struct DeviceError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

struct DataError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline void check(int rc, const char* what) {
    if (rc == SMK_OK) return;
    const std::string msg = std::string(what) + ": " + smk_last_error();
    if (rc == SMK_ERR_DATA) throw DataError(msg);
    throw DeviceError(msg);
}

using SgemmFn = void (*)(bool trans_a, bool trans_b, int M, int N, int K, float alpha, const float* A, int lda,
                         const float* B, int ldb, float beta, float* C, int ldc);
using Sgemm16Fn = void (*)(bool trans_b, int M, int N, int K, float alpha, const std::uint16_t* A, int lda,
                           const std::uint16_t* B, int ldb, float beta, float* C, int ldc);
using GemvQ8_0Fn = void (*)(int N, int K, const float* x, const std::uint8_t* Wq, float* y);
using GemvQ4_0Fn = void (*)(int N, int K, const float* x, const std::uint8_t* Wq, float* y);
using RowFn = void (*)(const float* in, float* out, int n);

struct KernelTable {
    const char* name;   // "gfx950"
    const char* flags;  // how the device code was built
    SgemmFn sgemm;
    Sgemm16Fn sgemm_f16;
    Sgemm16Fn sgemm_bf16;
    GemvQ8_0Fn gemv_q8_0;
    GemvQ4_0Fn gemv_q4_0;
    RowFn silu;
    RowFn softmax_row;
};

namespace detail {
inline void sgemm(bool ta, bool tb, int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                  float beta, float* C, int ldc) {
    check(smk_sgemm(ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc), "sgemm");
}
inline void sgemm_f16(bool tb, int M, int N, int K, float alpha, const std::uint16_t* A, int lda,
                      const std::uint16_t* B, int ldb, float beta, float* C, int ldc) {
    check(smk_sgemm_f16(tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc), "sgemm_f16");
}
inline void sgemm_bf16(bool tb, int M, int N, int K, float alpha, const std::uint16_t* A, int lda,
                       const std::uint16_t* B, int ldb, float beta, float* C, int ldc) {
    check(smk_sgemm_bf16(tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc), "sgemm_bf16");
}
inline void gemv_q8_0(int N, int K, const float* x, const std::uint8_t* Wq, float* y) {
    check(smk_gemv_q8_0(N, K, x, Wq, y), "gemv_q8_0");
}
inline void gemv_q4_0(int N, int K, const float* x, const std::uint8_t* Wq, float* y) {
    check(smk_gemv_q4_0(N, K, x, Wq, y), "gemv_q4_0");
}
inline void silu(const float* in, float* out, int n) { check(smk_silu(in, out, n), "silu"); }
inline void softmax_row(const float* in, float* out, int n) { check(smk_softmax(in, out, 1, n), "softmax"); }
}  // namespace detail

inline const KernelTable& kernels() {
    static const KernelTable t = {
        "gfx950",
        "hipcc --offload-arch=gfx950 -O3 -ffp-contract=off (packed FP32 off)",
        &detail::sgemm,
        &detail::sgemm_f16,
        &detail::sgemm_bf16,
        &detail::gemv_q8_0,
        &detail::gemv_q4_0,
        &detail::silu,
        &detail::softmax_row,
    };
    return t;
}

}  // namespace smk_host
