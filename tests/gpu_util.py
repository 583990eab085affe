"""Helpers of the GPU tests: device buffers through the library's own C ABI (no other
framework is loaded into the test process, so exactly one HIP runtime -- the one
libsmk_hip.so was built against -- is in use)."""

from __future__ import annotations

import numpy as np

from simd_ml_kernels import abi
from simd_ml_kernels.abi import Buffer


def dev(a: np.ndarray) -> Buffer:
    """A device copy of a numpy array (any dtype)."""
    return Buffer.of(a)


def empty(nbytes: int, fill: int = 0xEE) -> Buffer:
    """nbytes of device memory filled with `fill` (guard pattern)."""
    return Buffer.filled(nbytes, fill)


def host(buf: Buffer, dtype, count=None, offset: int = 0) -> np.ndarray:
    abi.call("smk_synchronize")
    return buf.numpy(dtype, count, offset)


def ptr(buf: Buffer, offset: int = 0) -> int:
    return buf.ptr + offset


def stream():
    return None  # the null stream


def call(name, *args):
    abi.call(name, *args)
