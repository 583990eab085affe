// bindings.cpp -- simd_ml_kernels._core for the MI355X: the reference's NumPy-facing API
// (src/bindings/pybind_entry.cpp, python/simd_ml_kernels/_core.pyi) on the gfx950 kernel table.
//
// Same entry names, argument lists and defaults, and the same error types: DTypeError
// (TypeError, RuntimeError) for a wrong dtype, ArgumentError (ValueError, RuntimeError) for a
// wrong shape / layout / value, raised here before any device work
// (pybind_entry.cpp:75-128, 944-961, 1082-1092).  Arrays are never converted; the GIL is
// released around every device call.  Device failures raise RuntimeError.
//
// Residency: a weight operand (Wq of gemv_*, B of a trans_b product) whose array is
// read-only all the way down its base chain -- a GGUF memmap opened mode="r" is -- is copied
// to the device once and reused (smk_weights_pin).  The module keeps a reference to that
// array, so its memory cannot be freed and reused while the device copy exists.  Writeable
// arrays (the llama example's KV cache, the bench's rotated copies) are uploaded per call.
//
// New entry points with no reference counterpart: rms_norm and rope (the example's numpy
// formulas, llama.py:184-187 / 169-178 / 387-396), gemm_q4_0 / gemm_q8_0 (batched decode),
// and the private _pin / _unpin / _pinned helpers.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>

#include <cstdlib>
#include <limits>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "kernel_table.hpp"

namespace py = pybind11;
using smk_host::kernels;

namespace {

struct DTypeError : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct ArgumentError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

constexpr int kQ4_0Bytes = 18, kQ8_0Bytes = 34;

bool is_f32(const py::array& a) { return a.dtype().kind() == 'f' && a.dtype().itemsize() == 4; }

void need_f32(const py::array& a, const char* name) {
    if (!is_f32(a))
        throw DTypeError(std::string(name) + " must be float32 (dtype=np.float32). Call arr.astype(np.float32) before passing.");
}

void need_contiguous(const py::array& a, const char* name) {
    if (!(a.flags() & py::array::c_style))
        throw ArgumentError(std::string(name) + " must be C-contiguous. Call numpy.ascontiguousarray(arr) before passing.");
}

void need_f32c(const py::array& a, const char* name) {
    need_f32(a, name);
    need_contiguous(a, name);
}

bool writeable(const py::array& a) { return a.writeable(); }

py::array_t<float> output_matrix(const py::object& C, py::ssize_t M, py::ssize_t N) {
    if (!py::isinstance<py::array>(C)) throw DTypeError("C must be a numpy.ndarray of dtype float32 (or None)");
    auto a = py::reinterpret_borrow<py::array>(C);
    need_f32c(a, "C");
    if (!writeable(a)) throw ArgumentError("C must be writeable. The array may be read-only; make a copy first.");
    if (a.ndim() != 2 || a.shape(0) != M || a.shape(1) != N)
        throw ArgumentError("C must have shape [" + std::to_string(M) + "×" + std::to_string(N) + "]");
    return py::reinterpret_borrow<py::array_t<float>>(a);
}

// ─── residency of read-only weights ──────────────────────────────────────────

std::mutex g_pin_mu;
// data pointer -> the array (kept alive).  Allocated once and never destroyed by C++: its
// references are dropped by an atexit hook while the interpreter still runs (a static map's
// destructor would run after Python has finalized and decrement without the GIL).
std::map<const void*, py::object>& g_pinned = *new std::map<const void*, py::object>();

size_t pin_budget() {
    static const size_t b = [] {
        const char* env = std::getenv("SMK_PIN_BUDGET_BYTES");
        return env ? static_cast<size_t>(std::strtoull(env, nullptr, 10)) : (static_cast<size_t>(160) << 30);
    }();
    return b;
}

// Read-only all the way down: every ndarray in the base chain is read-only.
bool immutable(const py::array& a) {
    if (writeable(a)) return false;
    py::object base = a.attr("base");
    for (int depth = 0; depth < 64 && !base.is_none(); ++depth) {
        if (py::isinstance<py::array>(base)) {
            if (writeable(py::reinterpret_borrow<py::array>(base))) return false;
        } else if (py::isinstance<py::bytearray>(base)) {
            return false;
        }
        if (!py::hasattr(base, "base")) break;
        base = base.attr("base");
    }
    return true;
}

// Pin arr's bytes on the device if it is immutable; called with the GIL held.
void maybe_pin(const py::array& arr, size_t nbytes) {
    if (nbytes == 0 || !immutable(arr)) return;
    const void* p = arr.data();
    {
        std::lock_guard<std::mutex> lk(g_pin_mu);
        if (g_pinned.count(p)) return;
    }
    size_t used = 0;
    smk_weights_stats(&used, nullptr);
    if (used + nbytes > pin_budget()) return;
    int rc;
    {
        py::gil_scoped_release release;
        rc = smk_weights_pin(p, nbytes);
    }
    if (rc == SMK_OK) {
        std::lock_guard<std::mutex> lk(g_pin_mu);
        g_pinned[p] = arr;
    }
    // On failure (e.g. out of device memory) the call still runs, uploading per call.
}

// ─── sgemm / sgemm_f16 / sgemm_bf16 ──────────────────────────────────────────

void check_isa(const std::string& isa) {
    if (isa.empty() || isa == kernels().name) return;
    if (isa == "scalar" || isa == "avx2" || isa == "avx512")
        throw std::runtime_error("isa='" + isa + "' was requested but this build does not include it. Use isa='' " +
                                 "(the kernels chosen for this device) or check simd_ml_kernels.build_info()['isa_usable'].");
    throw ArgumentError("isa must be one of: '', 'gfx950' (got '" + isa + "')");
}

py::array_t<float> new_c(py::ssize_t M, py::ssize_t N, float beta) {
    py::array_t<float> C({M, N});
    if (beta != 0.0f) std::fill(C.mutable_data(), C.mutable_data() + M * N, 0.0f);
    return C;
}

py::array_t<float> py_sgemm(py::array A, py::array B, py::object C, float alpha, float beta, const std::string& isa,
                            bool trans_a, bool trans_b) {
    check_isa(isa);
    need_f32c(A, "A");
    need_f32c(B, "B");
    if (A.ndim() != 2) throw ArgumentError("A must be 2-D");
    if (B.ndim() != 2) throw ArgumentError("B must be 2-D");
    const int lda = static_cast<int>(A.shape(1)), ldb = static_cast<int>(B.shape(1));
    const int M = static_cast<int>(A.shape(trans_a ? 1 : 0)), K = static_cast<int>(A.shape(trans_a ? 0 : 1));
    const int N = static_cast<int>(B.shape(trans_b ? 0 : 1)), Kb = static_cast<int>(B.shape(trans_b ? 1 : 0));
    if (Kb != K)
        throw ArgumentError("Shape mismatch: " + std::string(trans_a ? "A.T" : "A") + " is [" + std::to_string(M) + "×" +
                            std::to_string(K) + "] but " + (trans_b ? "B.T" : "B") + " is [" + std::to_string(Kb) +
                            "×" + std::to_string(N) + "]");
    py::array_t<float> Cout = C.is_none() ? new_c(M, N, beta) : output_matrix(C, M, N);
    if (trans_b && !trans_a) maybe_pin(B, static_cast<size_t>(B.nbytes()));
    const float* a = static_cast<const float*>(A.data());
    const float* b = static_cast<const float*>(B.data());
    float* c = Cout.mutable_data();
    {
        py::gil_scoped_release release;
        kernels().sgemm(trans_a, trans_b, M, N, K, alpha, a, lda, b, ldb, beta, c, N);
    }
    return Cout;
}

struct LowpShape {
    int M, N, K, ldb;
};

LowpShape lowp_shape(const py::array& A, const py::array& B, bool trans_b) {
    const int M = static_cast<int>(A.shape(0)), K = static_cast<int>(A.shape(1));
    const int N = static_cast<int>(B.shape(trans_b ? 0 : 1)), Kb = static_cast<int>(B.shape(trans_b ? 1 : 0));
    if (Kb != K)
        throw ArgumentError("Shape mismatch: A is [" + std::to_string(M) + "×" + std::to_string(K) + "] but " +
                            (trans_b ? "B.T" : "B") + " is [" + std::to_string(Kb) + "×" + std::to_string(N) + "]");
    return {M, N, K, static_cast<int>(B.shape(1))};
}

py::array_t<float> lowp_call(smk_host::Sgemm16Fn fn, py::array A, py::array B, float alpha, float beta, py::object C,
                             bool trans_b) {
    if (A.ndim() != 2) throw ArgumentError("A must be 2-D");
    if (B.ndim() != 2) throw ArgumentError("B must be 2-D");
    need_contiguous(A, "A");
    need_contiguous(B, "B");
    if (!trans_b)
        throw ArgumentError("this device build runs FP16/BF16 products with trans_b=True (x @ W.T, the decode GEMV) only");
    const LowpShape s = lowp_shape(A, B, trans_b);
    py::array_t<float> Cout = C.is_none() ? new_c(s.M, s.N, beta) : output_matrix(C, s.M, s.N);
    maybe_pin(B, static_cast<size_t>(B.nbytes()));
    const auto* a = static_cast<const uint16_t*>(A.data());
    const auto* b = static_cast<const uint16_t*>(B.data());
    float* c = Cout.mutable_data();
    {
        py::gil_scoped_release release;
        fn(trans_b, s.M, s.N, s.K, alpha, a, s.K, b, s.ldb, beta, c, s.N);
    }
    return Cout;
}

py::array_t<float> py_sgemm_f16(py::array A, py::array B, float alpha, float beta, py::object C, bool trans_b) {
    for (auto [arr, name] : {std::pair<py::array*, const char*>{&A, "A"}, {&B, "B"}})
        if (arr->dtype().kind() != 'f' || arr->dtype().itemsize() != 2)
            throw DTypeError(std::string(name) + " must be float16 (dtype=np.float16). Call arr.astype(np.float16) before passing.");
    return lowp_call(kernels().sgemm_f16, A, B, alpha, beta, C, trans_b);
}

py::array_t<float> py_sgemm_bf16(py::array A, py::array B, float alpha, float beta, py::object C, bool trans_b) {
    for (auto [arr, name] : {std::pair<py::array*, const char*>{&A, "A"}, {&B, "B"}}) {
        const auto dt = arr->dtype();
        if (dt.kind() == 'u' && dt.itemsize() == 2) continue;
        if (dt.itemsize() == 2 && py::str(dt.attr("name")).cast<std::string>() == "bfloat16") continue;
        std::string msg = std::string(name) + " must hold BF16 values: a uint16 array of BF16 bit patterns or an "
                          "ml_dtypes.bfloat16 array (got " + py::str(dt.attr("name")).cast<std::string>() + ").";
        if (dt.kind() == 'f' && dt.itemsize() == 2)
            msg += " float16 is IEEE half precision, not BF16: use sgemm_f16 for float16 inputs.";
        throw DTypeError(msg);
    }
    return lowp_call(kernels().sgemm_bf16, A, B, alpha, beta, C, trans_b);
}

// ─── elementwise ─────────────────────────────────────────────────────────────

py::array_t<float> py_silu(py::array x) {
    need_f32c(x, "x");
    py::array_t<float> out(x.request().shape);
    const float* in = static_cast<const float*>(x.data());
    float* o = out.mutable_data();
    const int n = static_cast<int>(x.size());
    {
        py::gil_scoped_release release;
        kernels().silu(in, o, n);
    }
    return out;
}

py::array_t<float> py_softmax(py::array x, int axis) {
    need_f32c(x, "x");
    if (x.ndim() < 1) throw ArgumentError("softmax requires an array with at least 1 dimension");
    const int nd = static_cast<int>(x.ndim());
    if (axis < 0) axis += nd;
    if (axis < 0 || axis >= nd) throw ArgumentError("softmax axis " + std::to_string(axis) + " out of range");
    if (axis != nd - 1)
        throw ArgumentError("softmax currently supports the last axis only (axis=-1). For other axes, transpose first.");
    py::array_t<float> out(x.request().shape);
    const int n = static_cast<int>(x.shape(nd - 1));
    const int rows = n ? static_cast<int>(x.size() / n) : 0;
    const float* in = static_cast<const float*>(x.data());
    float* o = out.mutable_data();
    int rc;
    {
        py::gil_scoped_release release;
        rc = smk_softmax(in, o, rows, n);
    }
    smk_host::check(rc, "softmax");
    return out;
}

py::array_t<float> py_rms_norm(py::array x, py::array weight, double eps) {
    need_f32c(x, "x");
    need_f32c(weight, "weight");
    if (x.ndim() < 1) throw ArgumentError("x must have at least 1 dimension");
    const py::ssize_t n = x.shape(x.ndim() - 1);
    if (weight.ndim() != 1 || weight.shape(0) != n)
        throw ArgumentError("weight must be 1-D with the last dimension of x (" + std::to_string(n) + ")");
    py::array_t<float> out(x.request().shape);
    const int rows = n ? static_cast<int>(x.size() / n) : 0;
    maybe_pin(weight, static_cast<size_t>(weight.nbytes()));
    const float* in = static_cast<const float*>(x.data());
    const float* w = static_cast<const float*>(weight.data());
    float* o = out.mutable_data();
    int rc;
    {
        py::gil_scoped_release release;
        rc = smk_rms_norm(in, w, o, rows, static_cast<int>(n), eps);
    }
    if (rc == SMK_ERR_ARGUMENT) throw ArgumentError(smk_last_error());
    smk_host::check(rc, "rms_norm");
    return out;
}

py::array_t<float> py_rope(py::array x, py::array cos, py::array sin, bool interleaved) {
    need_f32c(x, "x");
    need_f32c(cos, "cos");
    need_f32c(sin, "sin");
    if (x.ndim() != 2) throw ArgumentError("x must be 2-D [heads, head_dim]");
    const py::ssize_t hd = x.shape(1);
    if (hd % 2) throw ArgumentError("head_dim must be even");
    if (cos.ndim() != 1 || sin.ndim() != 1 || cos.shape(0) != hd || sin.shape(0) != hd)
        throw ArgumentError("cos and sin must be 1-D with head_dim = " + std::to_string(hd) + " elements");
    py::array_t<float> out(x.request().shape);
    const float* in = static_cast<const float*>(x.data());
    const float* c = static_cast<const float*>(cos.data());
    const float* s = static_cast<const float*>(sin.data());
    float* o = out.mutable_data();
    int rc;
    {
        py::gil_scoped_release release;
        rc = smk_rope(in, c, s, o, static_cast<int>(x.shape(0)), static_cast<int>(hd), interleaved ? 1 : 0);
    }
    smk_host::check(rc, "rope");
    return out;
}

// ─── quantize / gemv ─────────────────────────────────────────────────────────

py::array quantize_blocks(py::array W, int bb, int (*fn)(const float*, int, int, uint8_t*), const char* too_large) {
    need_f32c(W, "W");
    if (W.ndim() < 1) throw ArgumentError("W must have at least 1 dimension (rows of K values)");
    const py::ssize_t K = W.shape(W.ndim() - 1);
    if (K % 32 != 0)
        throw ArgumentError("K (the last dimension of W) must be a multiple of 32 (got " + std::to_string(K) + ")");
    if (K > std::numeric_limits<int>::max()) throw ArgumentError("K is too large");
    const py::ssize_t rows = K == 0 ? 0 : W.size() / K;
    if (rows > std::numeric_limits<int>::max()) throw ArgumentError("W has too many rows");
    std::vector<py::ssize_t> shape(W.shape(), W.shape() + W.ndim());
    shape.back() = K / 32 * bb;
    py::array_t<uint8_t> out(shape);
    const float* w = static_cast<const float*>(W.data());
    uint8_t* o = out.mutable_data();
    int rc;
    {
        py::gil_scoped_release release;
        rc = fn(w, static_cast<int>(rows), static_cast<int>(K), o);
    }
    if (rc == SMK_ERR_DATA) throw ArgumentError(too_large);
    smk_host::check(rc, "quantize");
    return std::move(out);
}

py::array py_quantize_q8_0(py::array W) {
    return quantize_blocks(W, kQ8_0Bytes, &smk_quantize_q8_0,
                           "W must be finite, with |W| below 127 * 65520 = 8321040 (a block scale max|w|/127 must fit float16)");
}

py::array py_quantize_q4_0(py::array W) {
    return quantize_blocks(W, kQ4_0Bytes, &smk_quantize_q4_0,
                           "W must be finite, with |W| below 8 * 65520 = 524160 (a block scale max|w|/8 must fit float16)");
}

void check_blocks(const py::array& Wq, py::ssize_t N, py::ssize_t K, int bb, const char* fmt) {
    const auto dt = Wq.dtype();
    if (dt.kind() != 'u' || dt.itemsize() != 1)
        throw DTypeError(std::string("Wq must be uint8 (blocks from quantize_") + fmt + "; dtype=np.uint8)");
    need_contiguous(Wq, "Wq");
    if (N < 0 || K < 0) throw ArgumentError("N and K must be >= 0");
    if (K % 32 != 0) throw ArgumentError("K must be a multiple of 32 (got " + std::to_string(K) + ")");
    if (N > std::numeric_limits<int>::max() || K > std::numeric_limits<int>::max())
        throw ArgumentError("N or K is too large");
    const py::ssize_t row = K / 32 * bb;
    if (Wq.size() != N * row)
        throw ArgumentError("Wq must hold N*K/32*" + std::to_string(bb) + " = " + std::to_string(N * row) +
                            " bytes (got " + std::to_string(Wq.size()) + ")");
}

py::array_t<float> gemv_blocks(py::array x, py::array Wq, py::ssize_t N, py::ssize_t K, int bb, const char* fmt,
                               smk_host::GemvQ4_0Fn gemv) {
    need_f32c(x, "x");
    check_blocks(Wq, N, K, bb, fmt);
    if (x.ndim() != 1 || x.shape(0) != K) throw ArgumentError("x must be 1-D with K = " + std::to_string(K) + " elements");
    py::array_t<float> y(N);
    maybe_pin(Wq, static_cast<size_t>(Wq.nbytes()));
    const float* xp = static_cast<const float*>(x.data());
    const uint8_t* wp = static_cast<const uint8_t*>(Wq.data());
    float* yp = y.mutable_data();
    {
        py::gil_scoped_release release;
        gemv(static_cast<int>(N), static_cast<int>(K), xp, wp, yp);
    }
    return y;
}

py::array_t<float> py_gemv_q8_0(py::array x, py::array Wq, py::ssize_t N, py::ssize_t K) {
    return gemv_blocks(x, Wq, N, K, kQ8_0Bytes, "q8_0", kernels().gemv_q8_0);
}

py::array_t<float> py_gemv_q4_0(py::array x, py::array Wq, py::ssize_t N, py::ssize_t K) {
    return gemv_blocks(x, Wq, N, K, kQ4_0Bytes, "q4_0", kernels().gemv_q4_0);
}

py::array_t<float> gemm_blocks(py::array X, py::array Wq, py::ssize_t N, py::ssize_t K, int bb, const char* fmt,
                               int (*fn)(int, int, int, const float*, const uint8_t*, float*)) {
    need_f32c(X, "X");
    check_blocks(Wq, N, K, bb, fmt);
    if (X.ndim() != 2 || X.shape(1) != K) throw ArgumentError("X must be 2-D [M, K] with K = " + std::to_string(K));
    const py::ssize_t M = X.shape(0);
    py::array_t<float> Y({M, N});
    maybe_pin(Wq, static_cast<size_t>(Wq.nbytes()));
    const float* xp = static_cast<const float*>(X.data());
    const uint8_t* wp = static_cast<const uint8_t*>(Wq.data());
    float* yp = Y.mutable_data();
    int rc;
    {
        py::gil_scoped_release release;
        rc = fn(static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), xp, wp, yp);
    }
    smk_host::check(rc, fmt);
    return Y;
}

// ─── build_info ──────────────────────────────────────────────────────────────

std::string device_name() {
    char name[256] = {0}, arch[64] = {0};
    int cus = 0;
    size_t hbm = 0;
    if (smk_device_info(name, sizeof name, arch, sizeof arch, &cus, &hbm) != SMK_OK) return "";
    return std::string(name) + " (" + arch + ", " + std::to_string(cus) + " CUs, " + std::to_string(hbm >> 30) + " GiB)";
}

py::dict build_info() {
    py::dict info;
    const std::string dev = device_name();
    info["isa_compiled"] = kernels().name;
    info["isa_usable"] = dev.empty() ? "" : kernels().name;
    py::dict flags;
    flags[kernels().name] = kernels().flags;
    info["isa_flags"] = flags;
    info["runtime_isa"] = kernels().name;
    info["kernel_flags"] = kernels().flags;
    info["version"] = "0.3.0";
    info["library"] = smk_version();
    info["openmp"] = false;
    info["q8_0_path"] = "gfx950_dot4";  // v_dot4_i32_i8 block sums, both Q8_0 and Q4_0
    info["gemv_device"] = dev;
    info["build_timestamp"] = std::string(__DATE__) + " " + __TIME__;
    return info;
}

int g_threads = 1;

}  // namespace

PYBIND11_MODULE(_core, m) {
    m.doc() =
        "simd-ml-kernels on AMD Instinct MI355X (gfx950): decode GEMV (Q4_0, Q8_0, FP16, BF16, FP32),\n"
        "SiLU, softmax, RMSNorm and RoPE on NumPy arrays, computed by hand-written HIP kernels.\n"
        "Arrays are never converted; read-only weight arrays stay resident in HBM after first use.";

    // Drop the resident arrays (and their device copies) at interpreter exit, with the GIL held.
    py::module_::import("atexit").attr("register")(py::cpp_function([]() {
        std::map<const void*, py::object> drop;
        {
            std::lock_guard<std::mutex> lk(g_pin_mu);
            drop.swap(g_pinned);
        }
        for (auto& kv : drop) smk_weights_unpin(kv.first);
    }));

    auto dtype_error = py::register_exception<DTypeError>(
        m, "DTypeError", py::make_tuple(py::handle(PyExc_TypeError), py::handle(PyExc_RuntimeError)));
    dtype_error.attr("__doc__") = "An array argument has the wrong dtype. Subclass of TypeError and RuntimeError.";
    auto argument_error = py::register_exception<ArgumentError>(
        m, "ArgumentError", py::make_tuple(py::handle(PyExc_ValueError), py::handle(PyExc_RuntimeError)));
    argument_error.attr("__doc__") =
        "An argument has the wrong shape, layout or value. Subclass of ValueError and RuntimeError.";
    py::register_exception<smk_host::DataError>(m, "_DataError", PyExc_RuntimeError);

    m.def("sgemm", &py_sgemm, py::arg("A"), py::arg("B"), py::arg("C") = py::none(), py::arg("alpha") = 1.0f,
          py::arg("beta") = 0.0f, py::arg("isa") = "", py::kw_only(), py::arg("trans_a") = false,
          py::arg("trans_b") = false,
          "C = alpha * op(A) @ op(B) + beta * C (float32). trans_b=True with few rows of A is the decode GEMV.");
    m.def("sgemm_f16", &py_sgemm_f16, py::arg("A"), py::arg("B"), py::arg("alpha") = 1.0f, py::arg("beta") = 0.0f,
          py::arg("C") = py::none(), py::kw_only(), py::arg("trans_b") = false,
          "float16 A and B (B [N, K] with trans_b), float32 accumulation and C.");
    m.def("sgemm_bf16", &py_sgemm_bf16, py::arg("A"), py::arg("B"), py::arg("alpha") = 1.0f, py::arg("beta") = 0.0f,
          py::arg("C") = py::none(), py::kw_only(), py::arg("trans_b") = false,
          "BF16 A and B (uint16 bit patterns), float32 accumulation and C.");
    m.def("silu", &py_silu, py::arg("x"), "x / (1 + exp(-x)), float32; |err| <= 1e-35 + 1e-6 |SiLU(x)|.");
    m.def("softmax", &py_softmax, py::arg("x"), py::arg("axis") = -1, "Softmax over the last axis, float32.");
    m.def("rms_norm", &py_rms_norm, py::arg("x"), py::arg("weight"), py::arg("eps") = 1e-5,
          "weight * x / sqrt(mean(x^2) + eps) over the last axis, bit-exact with the llama example's numpy formula.");
    m.def("rope", &py_rope, py::arg("x"), py::arg("cos"), py::arg("sin"), py::arg("interleaved") = true,
          "Rotary embedding of x [heads, head_dim] at one position (cos/sin [head_dim], halves equal).");
    m.def("quantize_q8_0", &py_quantize_q8_0, py::arg("W"), "float32 [..., K] -> GGUF Q8_0 blocks uint8 [..., K/32*34].");
    m.def("gemv_q8_0", &py_gemv_q8_0, py::arg("x"), py::arg("Wq"), py::arg("N"), py::arg("K"),
          "y = x @ W.T for W [N, K] as quantize_q8_0 blocks; float32 [N].");
    m.def("quantize_q4_0", &py_quantize_q4_0, py::arg("W"), "float32 [..., K] -> GGUF Q4_0 blocks uint8 [..., K/32*18].");
    m.def("gemv_q4_0", &py_gemv_q4_0, py::arg("x"), py::arg("Wq"), py::arg("N"), py::arg("K"),
          "y = x @ W.T for W [N, K] as quantize_q4_0 blocks; float32 [N].");
    m.def("gemm_q4_0", [](py::array X, py::array Wq, py::ssize_t N, py::ssize_t K) {
              return gemm_blocks(X, Wq, N, K, kQ4_0Bytes, "q4_0", &smk_gemm_q4_0);
          },
          py::arg("X"), py::arg("Wq"), py::arg("N"), py::arg("K"),
          "Y = X @ W.T for X [M, K]; row m equals gemv_q4_0(X[m], Wq, N, K) (each row quantized on its own).");
    m.def("gemm_q8_0", [](py::array X, py::array Wq, py::ssize_t N, py::ssize_t K) {
              return gemm_blocks(X, Wq, N, K, kQ8_0Bytes, "q8_0", &smk_gemm_q8_0);
          },
          py::arg("X"), py::arg("Wq"), py::arg("N"), py::arg("K"), "Y = X @ W.T for X [M, K], W as Q8_0 blocks.");
    m.def("build_info", &build_info, "Device, kernel table and build details.");
    m.def("detected_isa", []() { return std::string(kernels().name); }, "The kernel table every call uses: 'gfx950'.");
    m.def("set_num_threads", [](int n) {
              if (n <= 0) throw std::invalid_argument("num_threads must be positive");
              g_threads = n;
          },
          py::arg("n"), "Accepted for API compatibility; the device kernels do not use host threads.");
    m.def("get_num_threads", []() { return g_threads; });
    m.def("_set_isa", [](const std::string& isa) {
              if (isa == kernels().name) {
                  if (device_name().empty()) throw std::runtime_error("isa='" + isa + "' cannot run here: " + smk_last_error());
                  return;
              }
              if (isa == "scalar" || isa == "avx2" || isa == "avx512")
                  throw std::runtime_error("isa='" + isa + "' cannot run here (this build has the gfx950 table only)");
              throw ArgumentError("isa must be 'gfx950' (got '" + isa + "')");
          },
          py::arg("isa"), "Make this kernel table the active one (private; the selftest's loop).");
    m.def("_pin", [](py::array a) {
              const void* p = a.data();
              const size_t n = static_cast<size_t>(a.nbytes());  // (Python API: read with the GIL held)
              int rc;
              {
                  py::gil_scoped_release release;
                  rc = smk_weights_pin(p, n);
              }
              smk_host::check(rc, "pin");
              std::lock_guard<std::mutex> lk(g_pin_mu);
              g_pinned[p] = a;
          },
          py::arg("arr"), "Keep a device copy of arr for later calls (benchmarks). The caller must not modify arr.");
    m.def("_unpin", [](py::array a) {
              const void* p = a.data();
              int rc;
              {
                  py::gil_scoped_release release;  // waits for the calls that use the cached copy
                  rc = smk_weights_unpin(p);
              }
              smk_host::check(rc, "unpin");
              std::lock_guard<std::mutex> lk(g_pin_mu);
              g_pinned.erase(a.data());
          },
          py::arg("arr"));
    m.def("_unpin_all", []() {
              std::lock_guard<std::mutex> lk(g_pin_mu);
              for (auto& kv : g_pinned) smk_weights_unpin(kv.first);
              g_pinned.clear();
          });
    m.def("_pinned", []() {
              size_t bytes = 0;
              int n = 0;
              smk_weights_stats(&bytes, &n);
              return py::make_tuple(bytes, n);
          },
          "(bytes, entries) of device-resident weights.");
}
