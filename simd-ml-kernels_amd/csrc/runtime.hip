// runtime.hip -- the C ABI of libsmk_hip.so (include/smk_hip.h): device selection, per-thread
// streams and staging buffers, the device-resident weight cache, argument checks, and the
// host-pointer entry points that mirror the reference's KernelTable slots.
//
// Threading (the reference releases the GIL around every kernel and allows concurrent
// callers, pybind_entry.cpp:966-969, test_threads.cpp:168): every host thread gets its own
// stream and scratch, created on its first call; the weight cache is shared and guarded by a
// mutex.  A device copy in the cache is never freed while a call may read it: unpinning or
// eviction first synchronizes the device.
#include "abi_internal.hpp"
#include "launch.hpp"
#include "smk_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <shared_mutex>
#include <string>

namespace smk::abi {

namespace {
thread_local std::string t_error;
}  // namespace

const char* last_error() { return t_error.c_str(); }

int ok() {
    t_error.clear();
    return SMK_OK;
}

int fail(int code, const std::string& msg) {
    t_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    const int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? SMK_ERR_OUT_OF_MEMORY : SMK_ERR_DEVICE;
    return fail(code, std::string(what) + ": " + hipGetErrorString(e));
}

// ─── device ─────────────────────────────────────────────────────────────────

struct Device {
    int id = -1;
    int status = SMK_ERR_NO_DEVICE;
    std::string error;
    hipDeviceProp_t prop{};
};

Device& device() {
    static Device d = [] {
        Device r;
        int n = 0;
        const hipError_t e = hipGetDeviceCount(&n);
        if (e != hipSuccess || n <= 0) {
            r.error = std::string("no HIP device: ") + (e != hipSuccess ? hipGetErrorString(e) : "count is 0");
            return r;
        }
        int want = 0;
        if (const char* env = std::getenv("SMK_DEVICE")) want = std::atoi(env);
        if (want < 0 || want >= n) want = 0;
        if (hipGetDeviceProperties(&r.prop, want) != hipSuccess) {
            r.error = "hipGetDeviceProperties failed";
            return r;
        }
        if (std::strncmp(r.prop.gcnArchName, "gfx950", 6) != 0) {
            r.error = std::string("device ") + r.prop.gcnArchName + " is not gfx950 (this library is built for MI355X only)";
            return r;
        }
        // The code objects and the runtime ABI come from the build's ROCm; an older runtime
        // bound first in the process (another framework's bundled libamdhip64.so.7 has the
        // same SONAME) is refused rather than used.
        int rt = 0;
        if (hipRuntimeGetVersion(&rt) != hipSuccess || rt < HIP_VERSION) {
            r.error = "HIP runtime " + std::to_string(rt) + " is older than the one this library was built with (" +
                      std::to_string(HIP_VERSION) + "): load libsmk_hip.so before any library that bundles its own "
                      "HIP runtime";
            return r;
        }
        r.id = want;
        r.status = SMK_OK;
        smk::set_compute_units(r.prop.multiProcessorCount);
        return r;
    }();
    return d;
}

int use_device() {
    Device& d = device();
    if (d.status != SMK_OK) return fail(d.status, d.error);
    // Every entry point starts here: drop a stale error a failed call left in this thread's HIP
    // state, so that the launches of this call report their own status only.
    (void)hipGetLastError();
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != d.id) SMK_HIP(hipSetDevice(d.id), "hipSetDevice");
    return SMK_OK;
}

// Diagnostics settings of the quantized GEMV (smk_set_*): written under g_tuning_mu, read as a
// snapshot by every launch, so a setter running beside calls in flight never tears a read.
std::mutex g_tuning_mu;
smk::GemvTuning g_tuning;

smk::GemvTuning tuning_snapshot() {
    std::lock_guard<std::mutex> lk(g_tuning_mu);
    return g_tuning;
}

bool tuning_forced(const smk::GemvTuning& t) { return t.lanes_per_row || t.rows_per_wg || t.threads || t.unroll; }

// A launch refused under forced diagnostics settings: the settings do not fit this shape (LDS,
// lanes, rows) -- say so rather than report a bare launch error.  Out-of-memory keeps its code.
int gemv_launch_fail(hipError_t e, const smk::GemvTuning& t, int M, int N, int K) {
    if (e != hipErrorOutOfMemory && e != hipErrorMemoryAllocation && tuning_forced(t))
        return fail(SMK_ERR_ARGUMENT, std::string("gemv launch (") + hipGetErrorString(e) +
                                          "): the forced tuning (lanes_per_row " + std::to_string(t.lanes_per_row) +
                                          ", rows_per_wg " + std::to_string(t.rows_per_wg) + ", threads " +
                                          std::to_string(t.threads) + ", unroll " + std::to_string(t.unroll) +
                                          ") does not fit M=" + std::to_string(M) + " N=" + std::to_string(N) +
                                          " K=" + std::to_string(K) + "; smk_set_gemv_tuning(0, 0, 0, 0) restores "
                                          "the built-in choice");
    return hip_fail(e, "gemv launch");
}

int check_gemv_args(int M, int N, int K, const void* x, const void* W, const void* y) {
    if (M < 0 || N < 0 || K < 0) return fail(SMK_ERR_ARGUMENT, "M, N and K must be >= 0");
    if (K % 32) return fail(SMK_ERR_ARGUMENT, "K must be a multiple of 32");
    if (M > 0 && N > 0 && (!y || (K > 0 && (!x || !W)))) return fail(SMK_ERR_ARGUMENT, "null pointer");
    return SMK_OK;
}

}  // namespace smk::abi

namespace {

using namespace smk::abi;

// ─── per-thread context ─────────────────────────────────────────────────────

struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    hipError_t reserve(size_t n) {
        if (n <= cap) return hipSuccess;
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
        const size_t want = std::max<size_t>(n, 4096);
        const hipError_t e = hipMalloc(&p, want);
        if (e == hipSuccess) cap = want;
        return e;
    }
};

struct PinBuf {
    void* p = nullptr;
    size_t cap = 0;
    hipError_t reserve(size_t n) {
        if (n <= cap) return hipSuccess;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        cap = 0;
        const size_t want = std::max<size_t>(n, 4096);
        const hipError_t e = hipHostMalloc(&p, want, hipHostMallocDefault);
        if (e == hipSuccess) cap = want;
        return e;
    }
};

std::atomic<bool> g_exiting{false};

// Pinned staging: ha carries the first upload of a call (x or A), hb the second (C of a
// product with beta != 0), hc the download.  Each buffer is reused only after the stream has
// drained (every host-pointer call ends with a synchronizing download), so an upload still
// queued on the stream never sees its staging bytes overwritten by a later one of the same call.
struct Ctx {
    hipStream_t stream = nullptr;
    DevBuf a, b, c, w, flag;
    PinBuf ha, hb, hc;
    ~Ctx() {
        if (g_exiting.load()) return;  // the runtime may already be gone at process exit
        if (stream) (void)hipStreamDestroy(stream);
        for (DevBuf* d : {&a, &b, &c, &w, &flag})
            if (d->p) (void)hipFree(d->p);
        for (PinBuf* h : {&ha, &hb, &hc})
            if (h->p) (void)hipHostFree(h->p);
    }
};

thread_local Ctx t_ctx;

int context(Ctx** out) {
    if (const int rc = use_device()) return rc;
    if (!t_ctx.stream) {
        static std::once_flag once;
        std::call_once(once, [] { std::atexit([] { g_exiting.store(true); }); });
        SMK_HIP(hipStreamCreateWithFlags(&t_ctx.stream, hipStreamNonBlocking), "hipStreamCreate");
    }
    *out = &t_ctx;
    return SMK_OK;
}

// ─── weight cache ───────────────────────────────────────────────────────────

struct Entry {
    size_t bytes = 0;
    void* dev = nullptr;
};

// The weight cache.  Host-pointer calls hold g_cache_rw shared from their lookup until their
// result is downloaded (the device is done with the copy by then); pinning, replacing and
// unpinning take it exclusively, so a device copy is never freed under a call that uses it.
std::shared_mutex g_cache_rw;
std::map<uintptr_t, Entry> g_cache;  // keyed by host start address
size_t g_cache_bytes = 0;
using CacheUse = std::shared_lock<std::shared_mutex>;

// Device address of host range [p, p + n) if a pinned entry covers it, else nullptr.  The caller
// holds a CacheUse.
const void* cache_lookup(const void* p, size_t n) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    auto it = g_cache.upper_bound(a);
    if (it == g_cache.begin()) return nullptr;
    --it;
    if (a + n > it->first + it->second.bytes) return nullptr;
    return static_cast<const char*>(it->second.dev) + (a - it->first);
}

// Device copy of [p, p + n): the cached one, or an upload into the context's scratch.
int weights_on_device(Ctx* c, const void* p, size_t n, const void** dev) {
    if (n == 0) {
        *dev = nullptr;
        return SMK_OK;
    }
    if (const void* d = cache_lookup(p, n)) {
        *dev = d;
        return SMK_OK;
    }
    SMK_HIP(c->w.reserve(n), "device scratch for weights");
    SMK_HIP(hipMemcpyAsync(c->w.p, p, n, hipMemcpyHostToDevice, c->stream), "weights upload");
    *dev = c->w.p;
    return SMK_OK;
}

// Small host -> device copy through the pinned staging buffer `stage` (asynchronous: the
// caller must not reuse `stage` in the same call before the stream has run the copy).
int upload(Ctx* c, DevBuf& dst, const void* src, size_t n, PinBuf& stage) {
    SMK_HIP(dst.reserve(n), "device scratch");
    if (n == 0) return SMK_OK;
    SMK_HIP(stage.reserve(n), "pinned staging");
    std::memcpy(stage.p, src, n);
    SMK_HIP(hipMemcpyAsync(dst.p, stage.p, n, hipMemcpyHostToDevice, c->stream), "upload");
    return SMK_OK;
}
int upload(Ctx* c, DevBuf& dst, const void* src, size_t n) { return upload(c, dst, src, n, c->ha); }

// Device -> host through pinned staging; waits for the stream.
int download(Ctx* c, void* dst, const void* src, size_t n) {
    if (n == 0) {
        SMK_HIP(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        return SMK_OK;
    }
    SMK_HIP(c->hc.reserve(n), "pinned staging");
    SMK_HIP(hipMemcpyAsync(c->hc.p, src, n, hipMemcpyDeviceToHost, c->stream), "download");
    SMK_HIP(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    std::memcpy(dst, c->hc.p, n);
    return SMK_OK;
}

// Host-pointer quantized GEMV/GEMM: rows m < M of X [M, K] against W [N, K/32 blocks].
int host_gemm_quant(int bb, int M, int N, int K, const float* X, const uint8_t* Wq, float* Y) {
    if (const int rc = check_gemv_args(M, N, K, X, Wq, Y)) return rc;
    if (M == 0 || N == 0) return ok();
    if (K == 0) {
        std::fill(Y, Y + static_cast<size_t>(M) * N, 0.0f);
        return ok();
    }
    Ctx* c;
    if (const int rc = context(&c)) return rc;
    CacheUse use(g_cache_rw);
    const void* wd;
    if (const int rc = weights_on_device(c, Wq, static_cast<size_t>(N) * (K / 32) * bb, &wd)) return rc;
    const smk::GemvTuning tuning = tuning_snapshot();
    // Rows of X in uploads of at most 32 (one matrix-core launch at K <= 4096).
    for (int m0 = 0; m0 < M; m0 += 32) {
        const int mr = std::min(32, M - m0);
        if (const int rc = upload(c, c->a, X + static_cast<size_t>(m0) * K, static_cast<size_t>(mr) * K * 4)) return rc;
        SMK_HIP(c->c.reserve(static_cast<size_t>(mr) * N * 4), "device scratch");
        if (const hipError_t e = smk::gemv_quant(bb, mr, N, K, static_cast<const float*>(c->a.p), K,
                                                 static_cast<const uint8_t*>(wd), static_cast<float*>(c->c.p), N,
                                                 c->stream, &tuning);
            e != hipSuccess)
            return gemv_launch_fail(e, tuning, mr, N, K);
        if (const int rc = download(c, Y + static_cast<size_t>(m0) * N, c->c.p, static_cast<size_t>(mr) * N * 4))
            return rc;
    }
    return ok();
}

int host_quantize(int bb, const float* W, int N, int K, uint8_t* out) {
    if (N < 0 || K < 0 || K % 32) return fail(SMK_ERR_ARGUMENT, "N, K >= 0 and K % 32 == 0 required");
    if (N == 0 || K == 0) return ok();
    Ctx* c;
    if (const int rc = context(&c)) return rc;
    const size_t in_bytes = static_cast<size_t>(N) * K * 4, out_bytes = static_cast<size_t>(N) * (K / 32) * bb;
    SMK_HIP(c->a.reserve(in_bytes), "device scratch");
    SMK_HIP(c->c.reserve(out_bytes), "device scratch");
    SMK_HIP(c->flag.reserve(4), "device scratch");
    SMK_HIP(hipMemcpyAsync(c->a.p, W, in_bytes, hipMemcpyHostToDevice, c->stream), "upload");
    SMK_HIP(hipMemsetAsync(c->flag.p, 0, 4, c->stream), "memset");
    SMK_HIP(smk::quantize_weights(bb, N, K, static_cast<const float*>(c->a.p), static_cast<uint8_t*>(c->c.p),
                                  static_cast<int*>(c->flag.p), c->stream),
            "quantize launch");
    int bad = 0;
    SMK_HIP(hipMemcpyAsync(out, c->c.p, out_bytes, hipMemcpyDeviceToHost, c->stream), "download");
    SMK_HIP(hipMemcpyAsync(&bad, c->flag.p, 4, hipMemcpyDeviceToHost, c->stream), "download");
    SMK_HIP(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (bad) return fail(SMK_ERR_DATA, "W holds a NaN or infinity, or a block scale overflows float16");
    return ok();
}

// Host-pointer trans_b / general GEMM of element type elem (A and B in that type).
int host_gemm(int elem, bool ta, bool tb, int M, int N, int K, float alpha, const void* A, int lda, const void* B,
              int ldb, float beta, float* C, int ldc) {
    if (M < 0 || N < 0 || K < 0) return fail(SMK_ERR_ARGUMENT, "M, N and K must be >= 0");
    if (M == 0 || N == 0) return ok();
    const size_t es = elem == 0 ? 4 : 2;
    Ctx* c;
    if (const int rc = context(&c)) return rc;
    const size_t a_rows = ta ? K : M, b_rows = tb ? N : K;
    const size_t a_bytes = a_rows ? ((a_rows - 1) * lda + (ta ? M : K)) * es : 0;
    const size_t b_bytes = b_rows ? ((b_rows - 1) * ldb + (tb ? K : N)) * es : 0;
    const size_t c_bytes = ((static_cast<size_t>(M) - 1) * ldc + N) * 4;
    CacheUse use(g_cache_rw);
    if (K > 0) {
        if (const int rc = upload(c, c->a, A, a_bytes)) return rc;
    }
    const void* bd = nullptr;
    if (K > 0) {
        if (const int rc = weights_on_device(c, B, b_bytes, &bd)) return rc;
    }
    if (beta != 0.0f) {
        // C through its own staging buffer: A's upload from ha may not have run yet.
        if (const int rc = upload(c, c->c, C, c_bytes, c->hb)) return rc;
    } else {
        SMK_HIP(c->c.reserve(c_bytes), "device scratch");
    }
    float* cd = static_cast<float*>(c->c.p);
    if (elem == 0 && !(tb && !ta)) {
        SMK_HIP(smk::sgemm_generic(ta, tb, M, N, K, alpha, static_cast<const float*>(c->a.p), lda,
                                   static_cast<const float*>(bd), ldb, beta, cd, ldc, c->stream),
                "sgemm launch");
    } else if (tb) {
        SMK_HIP(smk::gemm_tb(elem, M, N, K, alpha, c->a.p, lda, bd, ldb, beta, cd, ldc, c->stream), "gemm launch");
    } else {
        return fail(SMK_ERR_ARGUMENT, "FP16/BF16 products without trans_b are not on this library's path");
    }
    return download(c, C, cd, c_bytes) ? SMK_ERR_DEVICE : ok();
}

}  // namespace

// ─── exported ABI ───────────────────────────────────────────────────────────

extern "C" {

const char* smk_last_error(void) { return smk::abi::last_error(); }

const char* smk_version(void) { return "simd-ml-kernels-amd 0.1.0 (gfx950)"; }

int smk_device_info(char* name, size_t name_len, char* arch, size_t arch_len, int* cus, size_t* hbm) {
    if (const int rc = use_device()) return rc;
    const Device& d = device();
    if (name && name_len) std::snprintf(name, name_len, "%s", d.prop.name);
    if (arch && arch_len) std::snprintf(arch, arch_len, "%s", d.prop.gcnArchName);
    if (cus) *cus = d.prop.multiProcessorCount;
    if (hbm) *hbm = d.prop.totalGlobalMem;
    return ok();
}

int smk_gemv_q4_0(int N, int K, const float* x, const uint8_t* Wq, float* y) {
    return host_gemm_quant(smk::kQ4_0Bytes, 1, N, K, x, Wq, y);
}
int smk_gemv_q8_0(int N, int K, const float* x, const uint8_t* Wq, float* y) {
    return host_gemm_quant(smk::kQ8_0Bytes, 1, N, K, x, Wq, y);
}
int smk_gemm_q4_0(int M, int N, int K, const float* X, const uint8_t* Wq, float* Y) {
    return host_gemm_quant(smk::kQ4_0Bytes, M, N, K, X, Wq, Y);
}
int smk_gemm_q8_0(int M, int N, int K, const float* X, const uint8_t* Wq, float* Y) {
    return host_gemm_quant(smk::kQ8_0Bytes, M, N, K, X, Wq, Y);
}

int smk_sgemm(int ta, int tb, int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
              float beta, float* C, int ldc) {
    return host_gemm(0, ta != 0, tb != 0, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
}
int smk_sgemm_f16(int tb, int M, int N, int K, float alpha, const uint16_t* A, int lda, const uint16_t* B, int ldb,
                  float beta, float* C, int ldc) {
    return host_gemm(1, false, tb != 0, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
}
int smk_sgemm_bf16(int tb, int M, int N, int K, float alpha, const uint16_t* A, int lda, const uint16_t* B, int ldb,
                   float beta, float* C, int ldc) {
    return host_gemm(2, false, tb != 0, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
}

int smk_silu(const float* in, float* out, int n) {
    if (n <= 0) return ok();
    Ctx* c;
    if (const int rc = context(&c)) return rc;
    if (const int rc = upload(c, c->a, in, static_cast<size_t>(n) * 4)) return rc;
    SMK_HIP(c->c.reserve(static_cast<size_t>(n) * 4), "device scratch");
    SMK_HIP(smk::silu(static_cast<const float*>(c->a.p), static_cast<float*>(c->c.p), n, c->stream), "silu launch");
    return download(c, out, c->c.p, static_cast<size_t>(n) * 4) ? SMK_ERR_DEVICE : ok();
}

int smk_softmax(const float* in, float* out, int rows, int n) {
    if (rows <= 0 || n <= 0) return ok();
    Ctx* c;
    if (const int rc = context(&c)) return rc;
    const size_t bytes = static_cast<size_t>(rows) * n * 4;
    if (const int rc = upload(c, c->a, in, bytes)) return rc;
    SMK_HIP(c->c.reserve(bytes), "device scratch");
    SMK_HIP(smk::softmax_rows(static_cast<const float*>(c->a.p), static_cast<float*>(c->c.p), rows, n, c->stream),
            "softmax launch");
    return download(c, out, c->c.p, bytes) ? SMK_ERR_DEVICE : ok();
}

int smk_quantize_q4_0(const float* W, int N, int K, uint8_t* out) { return host_quantize(smk::kQ4_0Bytes, W, N, K, out); }
int smk_quantize_q8_0(const float* W, int N, int K, uint8_t* out) { return host_quantize(smk::kQ8_0Bytes, W, N, K, out); }

int smk_rms_norm(const float* x, const float* w, float* y, int rows, int n, double eps) {
    if (rows <= 0 || n <= 0) return ok();
    if (rows < 0 || n < 0) return fail(SMK_ERR_ARGUMENT, "rms_norm: rows and n must be >= 0");
    Ctx* c;
    if (const int rc = context(&c)) return rc;
    const size_t bytes = static_cast<size_t>(rows) * n * 4;
    CacheUse use(g_cache_rw);
    if (const int rc = upload(c, c->a, x, bytes)) return rc;
    const void* wd;
    if (const int rc = weights_on_device(c, w, static_cast<size_t>(n) * 4, &wd)) return rc;
    SMK_HIP(c->c.reserve(bytes), "device scratch");
    SMK_HIP(smk::rms_norm(static_cast<const float*>(c->a.p), static_cast<const float*>(wd), static_cast<float*>(c->c.p),
                          rows, n, eps, c->stream),
            "rms_norm launch");
    return download(c, y, c->c.p, bytes) ? SMK_ERR_DEVICE : ok();
}

int smk_rope(const float* x, const float* cs, const float* sn, float* y, int heads, int hd, int interleaved) {
    if (heads <= 0 || hd <= 0) return ok();
    if (hd % 2) return fail(SMK_ERR_ARGUMENT, "rope: head_dim must be even");
    Ctx* c;
    if (const int rc = context(&c)) return rc;
    const size_t bytes = static_cast<size_t>(heads) * hd * 4;
    // x, cos and sin share one staging upload: [x | cos | sin].
    const size_t tb = bytes + 2 * static_cast<size_t>(hd) * 4;
    SMK_HIP(c->a.reserve(tb), "device scratch");
    SMK_HIP(c->ha.reserve(tb), "pinned staging");
    char* h = static_cast<char*>(c->ha.p);
    std::memcpy(h, x, bytes);
    std::memcpy(h + bytes, cs, static_cast<size_t>(hd) * 4);
    std::memcpy(h + bytes + hd * 4, sn, static_cast<size_t>(hd) * 4);
    SMK_HIP(hipMemcpyAsync(c->a.p, h, tb, hipMemcpyHostToDevice, c->stream), "upload");
    SMK_HIP(c->c.reserve(bytes), "device scratch");
    const float* d = static_cast<const float*>(c->a.p);
    SMK_HIP(smk::rope(d, d + static_cast<size_t>(heads) * hd, d + static_cast<size_t>(heads) * hd + hd,
                      static_cast<float*>(c->c.p), heads, hd, interleaved != 0, c->stream),
            "rope launch");
    return download(c, y, c->c.p, bytes) ? SMK_ERR_DEVICE : ok();
}

int smk_weights_pin(const void* host, size_t nbytes) {
    if (!host || nbytes == 0) return fail(SMK_ERR_ARGUMENT, "pin: empty range");
    if (const int rc = use_device()) return rc;
    {
        CacheUse use(g_cache_rw);
        auto it = g_cache.find(reinterpret_cast<uintptr_t>(host));
        if (it != g_cache.end() && it->second.bytes >= nbytes) return ok();
    }
    void* dev = nullptr;
    SMK_HIP(hipMalloc(&dev, nbytes), "pin: hipMalloc");
    const hipError_t e = hipMemcpy(dev, host, nbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail(e, "pin: upload");
    }
    std::unique_lock<std::shared_mutex> lk(g_cache_rw);  // waits for the calls using the cache
    auto it = g_cache.find(reinterpret_cast<uintptr_t>(host));
    if (it != g_cache.end()) {  // replaced by a larger range: device-pointer work may still read it
        (void)hipDeviceSynchronize();
        (void)hipFree(it->second.dev);
        g_cache_bytes -= it->second.bytes;
        g_cache.erase(it);
    }
    g_cache[reinterpret_cast<uintptr_t>(host)] = Entry{nbytes, dev};
    g_cache_bytes += nbytes;
    return ok();
}

int smk_weights_unpin(const void* host) {
    if (const int rc = use_device()) return rc;
    std::unique_lock<std::shared_mutex> lk(g_cache_rw);  // waits for the calls using the cache
    auto it = g_cache.find(reinterpret_cast<uintptr_t>(host));
    if (it == g_cache.end()) return ok();
    SMK_HIP(hipDeviceSynchronize(), "unpin: synchronize");
    SMK_HIP(hipFree(it->second.dev), "unpin: hipFree");
    g_cache_bytes -= it->second.bytes;
    g_cache.erase(it);
    return ok();
}

int smk_weights_stats(size_t* bytes, int* entries) {
    CacheUse use(g_cache_rw);
    if (bytes) *bytes = g_cache_bytes;
    if (entries) *entries = static_cast<int>(g_cache.size());
    return ok();
}

// ─── device-pointer entry points ────────────────────────────────────────────

static hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

static int d_gemm_quant(int bb, int M, int N, int K, const float* X, int ldx, const uint8_t* Wq, float* Y, int ldy,
                        void* stream) {
    if (const int rc = check_gemv_args(M, N, K, X, Wq, Y)) return rc;
    if (M > 0 && (ldx < K || ldy < N)) return fail(SMK_ERR_ARGUMENT, "ldx >= K and ldy >= N required");
    if (reinterpret_cast<uintptr_t>(X) % 4 || reinterpret_cast<uintptr_t>(Wq) % 2 || reinterpret_cast<uintptr_t>(Y) % 4)
        return fail(SMK_ERR_ARGUMENT, "X and Y must be 4-byte aligned and Wq 2-byte aligned");
    if (const int rc = use_device()) return rc;
    const smk::GemvTuning tuning = tuning_snapshot();
    if (const hipError_t e = smk::gemv_quant(bb, M, N, K, X, ldx, Wq, Y, ldy, S(stream), &tuning); e != hipSuccess)
        return gemv_launch_fail(e, tuning, M, N, K);
    return ok();
}

int smk_d_gemv_q4_0(int N, int K, const float* x, const uint8_t* Wq, float* y, void* stream) {
    return d_gemm_quant(smk::kQ4_0Bytes, 1, N, K, x, K, Wq, y, N, stream);
}
int smk_d_gemv_q8_0(int N, int K, const float* x, const uint8_t* Wq, float* y, void* stream) {
    return d_gemm_quant(smk::kQ8_0Bytes, 1, N, K, x, K, Wq, y, N, stream);
}
int smk_d_gemm_q4_0(int M, int N, int K, const float* X, int ldx, const uint8_t* Wq, float* Y, int ldy, void* stream) {
    return d_gemm_quant(smk::kQ4_0Bytes, M, N, K, X, ldx, Wq, Y, ldy, stream);
}
int smk_d_gemm_q8_0(int M, int N, int K, const float* X, int ldx, const uint8_t* Wq, float* Y, int ldy, void* stream) {
    return d_gemm_quant(smk::kQ8_0Bytes, M, N, K, X, ldx, Wq, Y, ldy, stream);
}

int smk_d_gemm_tb(int elem, int M, int N, int K, float alpha, const void* A, int lda, const void* B, int ldb,
                  float beta, float* C, int ldc, void* stream) {
    if (elem < 0 || elem > 2) return fail(SMK_ERR_ARGUMENT, "elem must be 0 (fp32), 1 (fp16) or 2 (bf16)");
    if (M < 0 || N < 0 || K < 0) return fail(SMK_ERR_ARGUMENT, "M, N and K must be >= 0");
    if (const int rc = use_device()) return rc;
    SMK_HIP(smk::gemm_tb(elem, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, S(stream)), "gemm launch");
    return ok();
}

int smk_d_sgemm(int ta, int tb, int M, int N, int K, float alpha, const float* A, int lda, const float* B, int ldb,
                float beta, float* C, int ldc, void* stream) {
    if (M < 0 || N < 0 || K < 0) return fail(SMK_ERR_ARGUMENT, "M, N and K must be >= 0");
    if (const int rc = use_device()) return rc;
    SMK_HIP(smk::sgemm_generic(ta != 0, tb != 0, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, S(stream)),
            "sgemm launch");
    return ok();
}

int smk_d_silu(const float* in, float* out, long long n, void* stream) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(smk::silu(in, out, n, S(stream)), "silu launch");
    return ok();
}

int smk_d_softmax(const float* in, float* out, int rows, int n, void* stream) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(smk::softmax_rows(in, out, rows, n, S(stream)), "softmax launch");
    return ok();
}

int smk_d_rms_norm(const float* x, const float* w, float* y, int rows, int n, double eps, void* stream) {
    if (rows < 0 || n < 0) return fail(SMK_ERR_ARGUMENT, "rms_norm: rows and n must be >= 0");
    if (const int rc = use_device()) return rc;
    SMK_HIP(smk::rms_norm(x, w, y, rows, n, eps, S(stream)), "rms_norm launch");
    return ok();
}

int smk_d_rope(const float* x, const float* cs, const float* sn, float* y, int heads, int hd, int interleaved,
               void* stream) {
    if (hd % 2) return fail(SMK_ERR_ARGUMENT, "rope: head_dim must be even");
    if (const int rc = use_device()) return rc;
    SMK_HIP(smk::rope(x, cs, sn, y, heads, hd, interleaved != 0, S(stream)), "rope launch");
    return ok();
}

int smk_d_quantize(int bb, long long rows, int K, const float* W, uint8_t* out, int* bad, void* stream) {
    if ((bb != smk::kQ4_0Bytes && bb != smk::kQ8_0Bytes) || rows < 0 || K < 0 || K % 32)
        return fail(SMK_ERR_ARGUMENT, "block_bytes 18 or 34, rows >= 0, K % 32 == 0 required");
    if (const int rc = use_device()) return rc;
    SMK_HIP(smk::quantize_weights(bb, rows, K, W, out, bad, S(stream)), "quantize launch");
    return ok();
}

int smk_d_quantize_x_q8(int K, const float* x, int8_t* qs, float* dx, int* bad, void* stream) {
    if (K < 0 || K % 32) return fail(SMK_ERR_ARGUMENT, "K % 32 == 0 required");
    if (const int rc = use_device()) return rc;
    SMK_HIP(smk::quantize_x_q8(K, x, qs, dx, bad, S(stream)), "quantize_x launch");
    return ok();
}

int smk_selfcheck_q8(unsigned* mismatches) {
    if (!mismatches) return fail(SMK_ERR_ARGUMENT, "null pointer");
    if (const int rc = use_device()) return rc;
    unsigned* d = nullptr;
    SMK_HIP(hipMalloc(&d, 2 * sizeof(unsigned)), "hipMalloc");
    hipError_t e = hipMemset(d, 0, 2 * sizeof(unsigned));
    if (e == hipSuccess) e = smk::q8_selfcheck(d, nullptr);
    if (e == hipSuccess) e = hipMemcpy(mismatches, d, 2 * sizeof(unsigned), hipMemcpyDeviceToHost);
    (void)hipFree(d);
    SMK_HIP(e, "q8 self-check");
    return ok();
}

int smk_d_block_sums(int bb, int N, int K, const int8_t* qs, const uint8_t* Wq, int32_t* out, void* stream) {
    if ((bb != smk::kQ4_0Bytes && bb != smk::kQ8_0Bytes) || N < 0 || K < 0 || K % 32)
        return fail(SMK_ERR_ARGUMENT, "block_bytes 18 or 34, N >= 0, K % 32 == 0 required");
    if (const int rc = use_device()) return rc;
    SMK_HIP(smk::block_sums(bb, N, K, qs, Wq, out, S(stream)), "block_sums launch");
    return ok();
}

int smk_d_read_roof(const void* src, size_t nbytes, float* sink, int nontemporal, void* stream) {
    if (reinterpret_cast<uintptr_t>(src) % 16) return fail(SMK_ERR_ARGUMENT, "src must be 16-byte aligned");
    if (const int rc = use_device()) return rc;
    SMK_HIP(smk::read_roof(src, nbytes, sink, nontemporal != 0, S(stream)), "read_roof launch");
    return ok();
}

int smk_d_copy(void* dst, const void* src, size_t nbytes, void* stream) {
    if (nbytes && (!dst || !src)) return fail(SMK_ERR_ARGUMENT, "null pointer");
    if (const int rc = use_device()) return rc;
    SMK_HIP(smk::copy_bytes(dst, src, nbytes, S(stream)), "copy launch");
    return ok();
}

int smk_malloc(void** p, size_t n) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipMalloc(p, n), "hipMalloc");
    return ok();
}
int smk_free(void* p) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipFree(p), "hipFree");
    return ok();
}
int smk_memcpy_h2d(void* dst, const void* src, size_t n) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipMemcpy(dst, src, n, hipMemcpyHostToDevice), "hipMemcpy");
    return ok();
}
int smk_memcpy_d2h(void* dst, const void* src, size_t n) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipMemcpy(dst, src, n, hipMemcpyDeviceToHost), "hipMemcpy");
    return ok();
}
int smk_memcpy_d2d(void* dst, const void* src, size_t n) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipMemcpy(dst, src, n, hipMemcpyDeviceToDevice), "hipMemcpy");
    return ok();
}
int smk_memset(void* p, int byte, size_t n) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipMemset(p, byte, n), "hipMemset");
    return ok();
}
int smk_synchronize(void) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return ok();
}

int smk_stream_create(void** s) {
    if (const int rc = use_device()) return rc;
    hipStream_t st = nullptr;
    SMK_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreate");
    *s = st;
    return ok();
}
int smk_stream_destroy(void* s) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipStreamDestroy(S(s)), "hipStreamDestroy");
    return ok();
}
int smk_stream_synchronize(void* s) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipStreamSynchronize(S(s)), "hipStreamSynchronize");
    return ok();
}
int smk_event_create(void** e) {
    if (const int rc = use_device()) return rc;
    hipEvent_t ev = nullptr;
    SMK_HIP(hipEventCreate(&ev), "hipEventCreate");
    *e = ev;
    return ok();
}
int smk_event_destroy(void* e) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipEventDestroy(static_cast<hipEvent_t>(e)), "hipEventDestroy");
    return ok();
}
int smk_event_record(void* e, void* s) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipEventRecord(static_cast<hipEvent_t>(e), S(s)), "hipEventRecord");
    return ok();
}
int smk_event_elapsed_ms(void* a, void* b, float* ms) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipEventSynchronize(static_cast<hipEvent_t>(b)), "hipEventSynchronize");
    SMK_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(a), static_cast<hipEvent_t>(b)), "hipEventElapsedTime");
    return ok();
}
int smk_graph_begin(void* s) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipStreamBeginCapture(S(s), hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    return ok();
}
int smk_graph_end(void* s, void** exec) {
    if (const int rc = use_device()) return rc;
    hipGraph_t graph = nullptr;
    SMK_HIP(hipStreamEndCapture(S(s), &graph), "hipStreamEndCapture");
    hipGraphExec_t ge = nullptr;
    const hipError_t e = hipGraphInstantiate(&ge, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    *exec = ge;
    return ok();
}
int smk_graph_launch(void* exec, void* s) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(exec), S(s)), "hipGraphLaunch");
    return ok();
}
int smk_graph_destroy(void* exec) {
    if (const int rc = use_device()) return rc;
    SMK_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec)), "hipGraphExecDestroy");
    return ok();
}
int smk_runtime_version(int* runtime, int* built) {
    if (built) *built = HIP_VERSION;
    if (runtime) {
        *runtime = 0;
        SMK_HIP(hipRuntimeGetVersion(runtime), "hipRuntimeGetVersion");
    }
    return ok();
}

int smk_set_q4_order(int reference_order) {
    if (reference_order != 0 && reference_order != 1) return fail(SMK_ERR_ARGUMENT, "reference_order must be 0 or 1");
    std::lock_guard<std::mutex> lk(g_tuning_mu);
    g_tuning.unordered = reference_order ? 0 : 1;
    return ok();
}

int smk_set_q4_stream(int mode) {
    if (mode < -1 || mode > 2) return fail(SMK_ERR_ARGUMENT, "mode must be -1, 0, 1 or 2");
    smk::set_q4_stream(mode);
    return ok();
}

int smk_set_q4_tiles(int tiles_in_flight) {
    if (tiles_in_flight != 0 && tiles_in_flight != -1 && (tiles_in_flight < 2 || tiles_in_flight > 4))
        return fail(SMK_ERR_ARGUMENT, "tiles_in_flight must be -1, 0, 2, 3 or 4");
    smk::set_q4_tiles(tiles_in_flight);
    return ok();
}

int smk_set_q4_mfma_min_rows(int rows) {
    if (rows < 0) return fail(SMK_ERR_ARGUMENT, "rows must be >= 0");
    std::lock_guard<std::mutex> lk(g_tuning_mu);
    g_tuning.mfma_min_rows = rows;
    return ok();
}

int smk_set_gemv_tuning(int lanes_per_row, int rows_per_wg, int threads, int unroll) {
    if (lanes_per_row != 0 && lanes_per_row != 8 && lanes_per_row != 16 && lanes_per_row != 32 && lanes_per_row != 64)
        return fail(SMK_ERR_ARGUMENT, "lanes_per_row must be 0, 8, 16, 32 or 64");
    if (rows_per_wg < 0) return fail(SMK_ERR_ARGUMENT, "rows_per_wg must be >= 0");
    if (threads != 0 && threads != 256 && threads != 512 && threads != 1024)
        return fail(SMK_ERR_ARGUMENT, "threads must be 0, 256, 512 or 1024");
    if (unroll != 0 && unroll != 1 && unroll != 2 && unroll != 4) return fail(SMK_ERR_ARGUMENT, "unroll must be 0, 1, 2 or 4");
    std::lock_guard<std::mutex> lk(g_tuning_mu);
    g_tuning.lanes_per_row = lanes_per_row;
    g_tuning.rows_per_wg = rows_per_wg;
    g_tuning.threads = threads;
    g_tuning.unroll = unroll;
    smk::set_lowp_tuning(lanes_per_row >= 16 ? lanes_per_row : 0, unroll);
    return ok();
}

const char* smk_gemv_path(int K, const void* Wq) {
    return smk::gemv_quant_path(0, 0, K, static_cast<const uint8_t*>(Wq));
}

}  // extern "C"
