"""ctypes binding of libsmk_hip.so's C ABI (include/smk_hip.h).

This is the binding a Python caller without the pybind11 module would write; the
tests and bench.py use it to drive the device-pointer entry points directly
(device buffers and streams can come from any allocator -- torch's, or
smk_malloc).  Every function returns an int status; ``check`` raises
RuntimeError with smk_last_error() on failure.
"""

from __future__ import annotations

import ctypes
import os
from functools import lru_cache

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lib", "libsmk_hip.so")

SMK_OK = 0
SMK_ERR_ARGUMENT = 1
SMK_ERR_NO_DEVICE = 2
SMK_ERR_DEVICE = 3
SMK_ERR_OUT_OF_MEMORY = 4
SMK_ERR_DATA = 5

_i, _ll, _f, _p, _sz = ctypes.c_int, ctypes.c_longlong, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t

class LlamaConfig(ctypes.Structure):
    """smk_llama_config of include/smk_hip.h."""
    _fields_ = [(n, ctypes.c_int) for n in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab",
                                            "matrix_type", "embed_type", "head_type", "rope_interleaved")] + \
               [("rms_eps", ctypes.c_double)]


# Tensor ids of smk_llama_set_tensor.
LLAMA_TENSORS = {"token_embd": 0, "output_norm": 1, "output": 2, "attn_norm": 3, "attn_q": 4, "attn_k": 5,
                 "attn_v": 6, "attn_output": 7, "ffn_norm": 8, "ffn_gate": 9, "ffn_up": 10, "ffn_down": 11}

# name -> argument types (all return int unless listed in _RESTYPE)
SIGNATURES = {
    "smk_last_error": [],
    "smk_version": [],
    "smk_device_info": [ctypes.c_char_p, _sz, ctypes.c_char_p, _sz, ctypes.POINTER(_i), ctypes.POINTER(_sz)],
    "smk_gemv_q4_0": [_i, _i, _p, _p, _p],
    "smk_gemv_q8_0": [_i, _i, _p, _p, _p],
    "smk_sgemm": [_i, _i, _i, _i, _i, _f, _p, _i, _p, _i, _f, _p, _i],
    "smk_sgemm_f16": [_i, _i, _i, _i, _f, _p, _i, _p, _i, _f, _p, _i],
    "smk_sgemm_bf16": [_i, _i, _i, _i, _f, _p, _i, _p, _i, _f, _p, _i],
    "smk_silu": [_p, _p, _i],
    "smk_softmax": [_p, _p, _i, _i],
    "smk_quantize_q4_0": [_p, _i, _i, _p],
    "smk_quantize_q8_0": [_p, _i, _i, _p],
    "smk_rms_norm": [_p, _p, _p, _i, _i, ctypes.c_double],
    "smk_rope": [_p, _p, _p, _p, _i, _i, _i],
    "smk_gemm_q4_0": [_i, _i, _i, _p, _p, _p],
    "smk_gemm_q8_0": [_i, _i, _i, _p, _p, _p],
    "smk_weights_pin": [_p, _sz],
    "smk_weights_unpin": [_p],
    "smk_weights_stats": [ctypes.POINTER(_sz), ctypes.POINTER(_i)],
    "smk_d_gemv_q4_0": [_i, _i, _p, _p, _p, _p],
    "smk_d_gemv_q8_0": [_i, _i, _p, _p, _p, _p],
    "smk_d_gemm_q4_0": [_i, _i, _i, _p, _i, _p, _p, _i, _p],
    "smk_d_gemm_q4_0_noalloc": [_i, _i, _i, _p, _i, _p, _p, _i, _p],
    "smk_d_gemm_q8_0": [_i, _i, _i, _p, _i, _p, _p, _i, _p],
    "smk_d_gemm_tb": [_i, _i, _i, _i, _f, _p, _i, _p, _i, _f, _p, _i, _p],
    "smk_d_sgemm": [_i, _i, _i, _i, _i, _f, _p, _i, _p, _i, _f, _p, _i, _p],
    "smk_d_silu": [_p, _p, _ll, _p],
    "smk_d_softmax": [_p, _p, _i, _i, _p],
    "smk_d_rms_norm": [_p, _p, _p, _i, _i, ctypes.c_double, _p],
    "smk_d_rope": [_p, _p, _p, _p, _i, _i, _i, _p],
    "smk_d_quantize": [_i, _ll, _i, _p, _p, _p, _p],
    "smk_d_quantize_x_q8": [_i, _p, _p, _p, _p, _p],
    "smk_d_block_sums": [_i, _i, _i, _p, _p, _p, _p],
    "smk_selfcheck_q8": [_p],
    "smk_d_read_roof": [_p, _sz, _p, _i, _p],
    "smk_d_copy": [_p, _p, _sz, _p],
    "smk_llama_create": [_p, ctypes.POINTER(_p)],
    "smk_llama_destroy": [_p],
    "smk_llama_set_tensor": [_p, _i, _i, _p, _sz],
    "smk_llama_reset": [_p, _i, _p, _p],
    "smk_llama_step": [_p, _i, _p],
    "smk_llama_generate": [_p, _p, _i, _i, _p, _p],
    "smk_llama_info": [_p, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(ctypes.c_ulonglong)],
    "smk_llama_step_profile": [_p, _i, _p, _p, _i],
    "smk_llama_set_prefill_rows": [_p, _i],
    "smk_malloc": [ctypes.POINTER(_p), _sz],
    "smk_free": [_p],
    "smk_memcpy_h2d": [_p, _p, _sz],
    "smk_memcpy_d2h": [_p, _p, _sz],
    "smk_memcpy_d2d": [_p, _p, _sz],
    "smk_memset": [_p, _i, _sz],
    "smk_synchronize": [],
    "smk_stream_create": [ctypes.POINTER(_p)],
    "smk_stream_destroy": [_p],
    "smk_stream_synchronize": [_p],
    "smk_event_create": [ctypes.POINTER(_p)],
    "smk_event_destroy": [_p],
    "smk_event_record": [_p, _p],
    "smk_event_elapsed_ms": [_p, _p, ctypes.POINTER(_f)],
    "smk_graph_begin": [_p],
    "smk_graph_end": [_p, ctypes.POINTER(_p)],
    "smk_graph_launch": [_p, _p],
    "smk_graph_destroy": [_p],
    "smk_runtime_version": [ctypes.POINTER(_i), ctypes.POINTER(_i)],
    "smk_set_gemv_tuning": [_i, _i, _i, _i],
    "smk_set_q4_order": [_i],
    "smk_set_q4_stream": [_i],
    "smk_set_q4_tiles": [_i],
    "smk_set_q4_mfma_min_rows": [_i],
    "smk_gemv_path": [_i, _p],
}
_RESTYPE = {"smk_last_error": ctypes.c_char_p, "smk_version": ctypes.c_char_p, "smk_gemv_path": ctypes.c_char_p}


@lru_cache(maxsize=None)
def lib(path: str = LIB) -> ctypes.CDLL:
    """Load libsmk_hip.so and declare every entry point of smk_hip.h."""
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} missing: run `make -C simd-ml-kernels_amd`")
    L = ctypes.CDLL(path)
    for name, args in SIGNATURES.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    return L


def check(rc: int, what: str = "smk") -> None:
    if rc != SMK_OK:
        raise RuntimeError(f"{what}: status {rc}: {lib().smk_last_error().decode()}")


def call(name: str, *args) -> None:
    """lib().<name>(*args), raising on a non-zero status."""
    check(getattr(lib(), name)(*args), name)


# ─── small RAII helpers over the ABI's device objects ──────────────────────


class Buffer:
    """A device allocation (smk_malloc), freed with the object."""

    def __init__(self, nbytes: int):
        p = ctypes.c_void_p()
        call("smk_malloc", ctypes.byref(p), max(int(nbytes), 1))
        self.ptr, self.nbytes = p.value, int(nbytes)

    @classmethod
    def of(cls, a) -> "Buffer":
        """A device copy of a numpy array."""
        import numpy as np
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            call("smk_memcpy_h2d", b.ptr, a.ctypes.data, a.nbytes)
        return b

    @classmethod
    def filled(cls, nbytes: int, byte: int = 0) -> "Buffer":
        b = cls(nbytes)
        call("smk_memset", b.ptr, byte, max(int(nbytes), 1))
        return b

    def numpy(self, dtype, count: int | None = None, offset: int = 0):
        """Copy device bytes [offset, ...) back as a numpy array of dtype."""
        import numpy as np
        dt = np.dtype(dtype)
        n = (self.nbytes - offset) // dt.itemsize if count is None else int(count)
        out = np.empty(n, dt)
        if n:
            call("smk_memcpy_d2h", out.ctypes.data, self.ptr + offset, n * dt.itemsize)
        return out

    def __del__(self):
        if getattr(self, "ptr", None):
            lib().smk_free(self.ptr)
            self.ptr = None


class Stream:
    def __init__(self):
        p = ctypes.c_void_p()
        call("smk_stream_create", ctypes.byref(p))
        self.handle = p.value

    def synchronize(self):
        call("smk_stream_synchronize", self.handle)

    def __del__(self):
        if getattr(self, "handle", None):
            lib().smk_stream_destroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        call("smk_event_create", ctypes.byref(p))
        self.handle = p.value

    def record(self, stream: "Stream | None" = None):
        call("smk_event_record", self.handle, stream.handle if stream else None)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        call("smk_event_elapsed_ms", self.handle, end.handle, ctypes.byref(ms))
        return float(ms.value)

    def __del__(self):
        if getattr(self, "handle", None):
            lib().smk_event_destroy(self.handle)
            self.handle = None


class Graph:
    """Work enqueued on `stream` inside ``with Graph.capture(stream) as g:`` becomes one graph."""

    def __init__(self, handle):
        self.handle = handle

    @staticmethod
    def capture(stream: Stream):
        return _Capture(stream)

    def launch(self, stream: Stream):
        call("smk_graph_launch", self.handle, stream.handle)

    def __del__(self):
        if getattr(self, "handle", None):
            lib().smk_graph_destroy(self.handle)
            self.handle = None


class _Capture:
    def __init__(self, stream: Stream):
        self.stream, self.graph = stream, None

    def __enter__(self):
        call("smk_graph_begin", self.stream.handle)
        return self

    def __exit__(self, *exc):
        p = ctypes.c_void_p()
        call("smk_graph_end", self.stream.handle, ctypes.byref(p))
        self.graph = Graph(p.value)
        return False
