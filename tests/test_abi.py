"""CPU checks of the boundary: the C-ABI library loads and exports every symbol that
include/smk_hip.h declares, the ctypes table covers them, and the pybind11 module's
argument validation raises the reference's error types before any device work
(pybind_entry.cpp:75-128, 944-961; test_bindings_edge_cases.py:651-743).  No test
here launches a kernel."""

import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "smk_hip.h")
LIB = os.path.join(ROOT, "simd-ml-kernels_amd", "lib", "libsmk_hip.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(smk_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "smk_gemv_q4_0" in names and "smk_d_gemv_q4_0" in names and len(names) >= 40


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (smk_\w+)", out))
    missing = [n for n in declared() if n not in exported]
    assert not missing, missing


def test_code_objects_have_no_packed_fp32_and_no_scratch():
    """The built gfx950 code objects (simd-ml-kernels_amd/check_objects.py, also run at link
    time): no packed-FP32 add/mul/fma instruction and no kernel with a private segment."""
    build = os.path.join(ROOT, "simd-ml-kernels_amd", "build")
    if not os.path.isdir(build) or not any(f.endswith(".o") for f in os.listdir(build)):
        pytest.skip("no build/ objects (the library was built elsewhere)")
    r = subprocess.run(["python3", os.path.join(ROOT, "simd-ml-kernels_amd", "check_objects.py"), build],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "clean" in r.stdout


def test_ctypes_table_matches_header():
    from simd_ml_kernels import abi
    assert sorted(abi.SIGNATURES) == declared()
    L = abi.lib()
    for n in declared():
        assert getattr(L, n) is not None
    assert L.smk_version().decode().startswith("simd-ml-kernels-amd")


def test_module_imports_with_reference_names():
    import simd_ml_kernels as sk
    for name in ("gemv_q4_0", "gemv_q8_0", "quantize_q4_0", "quantize_q8_0", "sgemm", "sgemm_f16", "sgemm_bf16",
                 "silu", "softmax", "rms_norm", "rope", "gemm_q4_0", "build_info", "detected_isa"):
        assert callable(getattr(sk, name))
    assert issubclass(sk.DTypeError, TypeError) and issubclass(sk.DTypeError, RuntimeError)
    assert issubclass(sk.ArgumentError, ValueError) and issubclass(sk.ArgumentError, RuntimeError)
    assert sk.detected_isa() == "gfx950"


class TestValidation:
    """Rejected inputs of gemv / quantize / sgemm (test_bindings_edge_cases.py:651-743)."""

    @pytest.fixture
    def sk(self):
        import simd_ml_kernels as sk
        return sk

    @pytest.mark.parametrize("fmt,bb", [("q4_0", 18), ("q8_0", 34)])
    def test_gemv_rejections(self, sk, fmt, bb):
        gemv = getattr(sk, f"gemv_{fmt}")
        x = np.ones(64, np.float32)
        wq = np.zeros(3 * 2 * bb, np.uint8)
        with pytest.raises(sk.DTypeError):
            gemv(x.astype(np.float64), wq, 3, 64)
        with pytest.raises(sk.DTypeError):
            gemv(x, wq.astype(np.int8), 3, 64)
        with pytest.raises(sk.ArgumentError):
            gemv(x, wq, 3, 60)                       # K % 32
        with pytest.raises(sk.ArgumentError):
            gemv(x, wq, -1, 64)
        with pytest.raises(sk.ArgumentError):
            gemv(x[:32], wq, 3, 64)                  # x length
        with pytest.raises(sk.ArgumentError):
            gemv(x, wq[:-1], 3, 64)                  # Wq size
        with pytest.raises(sk.ArgumentError):
            gemv(x, np.zeros((3 * 2 * bb, 2), np.uint8)[:, 0], 3, 64)  # not contiguous
        with pytest.raises(sk.ArgumentError):
            gemv(np.ones((64, 2), np.float32)[:, 0], wq, 3, 64)

    @pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
    def test_quantize_rejections(self, sk, fmt):
        q = getattr(sk, f"quantize_{fmt}")
        with pytest.raises(sk.DTypeError):
            q(np.ones((2, 64), np.float64))
        with pytest.raises(sk.ArgumentError):
            q(np.ones((2, 48), np.float32))
        with pytest.raises(sk.ArgumentError):
            q(np.ones((64, 2), np.float32).T)

    def test_sgemm_rejections(self, sk):
        A = np.ones((2, 8), np.float32)
        with pytest.raises(sk.DTypeError):
            sk.sgemm(A.astype(np.float64), A, trans_b=True)
        with pytest.raises(sk.ArgumentError):
            sk.sgemm(A, np.ones((3, 7), np.float32), trans_b=True)
        with pytest.raises(sk.ArgumentError):
            sk.sgemm(A, A, C=np.zeros((2, 3), np.float32), trans_b=True)
        with pytest.raises(RuntimeError):
            sk.sgemm(A, A, isa="avx2", trans_b=True)
        with pytest.raises(sk.ArgumentError):
            sk.sgemm(A, A, isa="nope", trans_b=True)
        with pytest.raises(sk.DTypeError):
            sk.sgemm_f16(A, A, trans_b=True)
        with pytest.raises(sk.DTypeError):
            sk.sgemm_bf16(A.astype(np.float16), A.astype(np.float16), trans_b=True)

    def test_rms_norm_and_rope_rejections(self, sk):
        with pytest.raises(sk.ArgumentError):
            sk.rms_norm(np.ones(8, np.float32), np.ones(7, np.float32))
        with pytest.raises(sk.ArgumentError):
            sk.rope(np.ones((2, 7), np.float32), np.ones(7, np.float32), np.ones(7, np.float32))
        with pytest.raises(sk.ArgumentError):
            sk.rope(np.ones((2, 8), np.float32), np.ones(6, np.float32), np.ones(8, np.float32))
