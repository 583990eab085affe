"""simd-ml-kernels on AMD Instinct MI355X (gfx950).

The reference's NumPy-facing API for the decode path -- quantize_q4_0 / gemv_q4_0,
quantize_q8_0 / gemv_q8_0, sgemm / sgemm_f16 / sgemm_bf16 with ``trans_b=True``
(the decode GEMV), silu and softmax -- plus rms_norm, rope and the batched
gemm_q4_0 / gemm_q8_0, all computed by hand-written HIP kernels through
libsmk_hip.so (include/smk_hip.h).  The compiled extension is
``simd_ml_kernels._core``; this module re-exports its public API.

There is no CPU fallback: if the extension or the HIP library is missing the
import fails, and without a gfx950 device every call raises RuntimeError.
"""

try:
    from ._core import (
        ArgumentError,
        DTypeError,
        build_info,
        detected_isa,
        gemm_q4_0,
        gemm_q8_0,
        gemv_q4_0,
        gemv_q8_0,
        get_num_threads,
        quantize_q4_0,
        quantize_q8_0,
        rms_norm,
        rope,
        set_num_threads,
        sgemm,
        sgemm_bf16,
        sgemm_f16,
        silu,
        softmax,
    )
except ImportError as exc:  # pragma: no cover - the build is part of the product
    raise ImportError(
        "simd_ml_kernels._core (the MI355X extension) is not built: run "
        "`make -C simd-ml-kernels_amd` or __graft_entry__.build()") from exc

__version__ = "0.3.0"

__all__ = [
    "ArgumentError",
    "DTypeError",
    "build_info",
    "detected_isa",
    "gemm_q4_0",
    "gemm_q8_0",
    "gemv_q4_0",
    "gemv_q8_0",
    "get_num_threads",
    "quantize_q4_0",
    "quantize_q8_0",
    "rms_norm",
    "rope",
    "set_num_threads",
    "sgemm",
    "sgemm_bf16",
    "sgemm_f16",
    "silu",
    "softmax",
]
