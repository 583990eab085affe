// noalloc.hip -- the batched Q4_0 product with a library-held scratch array, for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc): smk_d_gemm_q4_0_noalloc.
//
// smk_d_gemm_q4_0 (several rows of x on the int8 matrix cores) quantizes x into a scratch buffer
// it allocates per (stream, host thread) on first use and grows on demand.  This entry point
// runs the same kernels, bit for bit, on a fixed array instead: `scratch`, kScratchBytes of
// device memory in the library's code object, one copy per GPU the library runs on, held until
// the process ends.  Its device address is looked up once per device (hipGetSymbolAddress on the
// first call made with that device current) and only that address is used from host code.
// Nothing in it must start at zero: each call's quantizer writes every byte that call's stored
// outputs read (rows of a launch past M read stale bytes, and their products are never stored).
// Every call on a GPU shares that GPU's array: calls that overlap on one GPU (two streams, two
// host threads) race and must be serialized by the caller.
#include "abi_internal.hpp"
#include "launch.hpp"
#include "smk_hip.h"

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

namespace {

constexpr size_t kScratchBytes = size_t(4) << 20;  // the x image of up to 256 rows of x at K = 14336

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on the first call with that device).
int scratch_address(void** out) {
    int dev = 0;
    SMK_HIP(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return smk::abi::fail(SMK_ERR_DEVICE, "device index out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        SMK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return SMK_OK;
}

}  // namespace

extern "C" int smk_d_gemm_q4_0_noalloc(int M, int N, int K, const float* X, int ldx, const uint8_t* Wq, float* Y,
                                       int ldy, void* stream) {
    using namespace smk::abi;
    if (const int rc = check_gemv_args(M, N, K, X, Wq, Y)) return rc;
    if (M > 0 && (ldx < K || ldy < N)) return fail(SMK_ERR_ARGUMENT, "ldx >= K and ldy >= N required");
    if (reinterpret_cast<uintptr_t>(X) % 4 || reinterpret_cast<uintptr_t>(Wq) % 2 || reinterpret_cast<uintptr_t>(Y) % 4)
        return fail(SMK_ERR_ARGUMENT, "X and Y must be 4-byte aligned and Wq 2-byte aligned");
    const size_t need = M > 0 && K > 0 ? smk::gemm_q4_mfma_workspace(M, K) : 0;
    if (need > kScratchBytes)
        return fail(SMK_ERR_ARGUMENT, "smk_d_gemm_q4_0_noalloc: M=" + std::to_string(M) + " rows of K=" +
                                          std::to_string(K) + " need " + std::to_string(need) +
                                          " bytes of scratch; its array holds " + std::to_string(kScratchBytes) +
                                          " (split the rows into several calls)");
    if (const int rc = use_device()) return rc;
    void* ws = nullptr;
    if (const int rc = scratch_address(&ws)) return rc;
    smk::GemvTuning t = tuning_snapshot();
    t.workspace = ws;
    t.workspace_bytes = kScratchBytes;
    if (const hipError_t e = smk::gemv_quant(smk::kQ4_0Bytes, M, N, K, X, ldx, Wq, Y, ldy,
                                             static_cast<hipStream_t>(stream), &t);
        e != hipSuccess)
        return gemv_launch_fail(e, t, M, N, K);
    return ok();
}
