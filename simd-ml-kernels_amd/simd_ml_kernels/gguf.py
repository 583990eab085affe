"""GGUF model files (llama.cpp's format, versions 2 and 3) for the decode engine: a reader that
maps the file once and hands out every tensor as a read-only numpy view of the mapping, and a
writer for the synthetic models of the decode benchmark.

Everything in a GGUF file is little-endian:

* header -- the four bytes "GGUF", the format version (uint32), the number of tensors (uint64)
  and the number of key/value pairs (uint64);
* key/value pairs -- a string key, a uint32 value kind, then the value.  A string is a uint64
  byte count followed by UTF-8 bytes.  Kinds 0-7 and 10-12 are fixed-size scalars (see
  _SCALAR), 8 is a string, 9 an array: uint32 element kind, uint64 element count, elements;
* tensor directory -- per tensor: string name, uint32 rank, `rank` uint64 extents listed
  fastest-varying first, uint32 ggml element type, uint64 offset within the data section;
* data section -- begins at the first multiple of the `general.alignment` value (32 when the
  key is absent) past the directory.

Tensors of type F32 / F16 / BF16 / Q8_0 / Q4_0 are served (what the example decode loop,
examples/llama/gguf_reader.py:39-129, reads).  A quantized tensor is its raw blocks,
uint8 [rows, K/32 * block_bytes] -- the bytes gemv_q4_0 / gemv_q8_0 take; BF16 is uint16 bits.
"""

from __future__ import annotations

import json
import os
import struct
from typing import Iterable

import numpy as np

F32, F16, Q4_0, Q8_0, BF16 = 0, 1, 2, 8, 30
# ggml element type -> (label, bytes per block, values per block).
GGML_TYPES = {F32: ("F32", 4, 1), F16: ("F16", 2, 1), BF16: ("BF16", 2, 1), Q4_0: ("Q4_0", 18, 32),
              Q8_0: ("Q8_0", 34, 32)}

# Value kinds of the key/value section.
_STRING, _ARRAY = 8, 9
_SCALAR = {0: np.dtype("u1"), 1: np.dtype("i1"), 2: np.dtype("<u2"), 3: np.dtype("<i2"), 4: np.dtype("<u4"),
           5: np.dtype("<i4"), 6: np.dtype("<f4"), 7: np.dtype("?"), 10: np.dtype("<u8"), 11: np.dtype("<i8"),
           12: np.dtype("<f8")}
_BOOL, _U32, _I32, _F32, _U64, _I64, _F64 = 7, 4, 5, 6, 10, 11, 12


def type_label(ggml_type: int) -> str:
    entry = GGML_TYPES.get(ggml_type)
    return entry[0] if entry else f"ggml type {ggml_type}"


def tensor_bytes(ggml_type: int, shape: Iterable[int]) -> int:
    """Bytes of a tensor of `shape` (outermost first) stored as `ggml_type`."""
    dims = [int(d) for d in shape]
    _, block_bytes, block_values = GGML_TYPES[ggml_type]
    if dims[-1] % block_values:
        raise ValueError(f"a row of {dims[-1]} values does not split into blocks of {block_values}")
    n_rows = 1
    for d in dims[:-1]:
        n_rows *= d
    return n_rows * (dims[-1] // block_values) * block_bytes


class Tensor:
    """One tensor of a GGUF file: its name, ggml element type, shape (outermost first, [N, K] for
    a weight matrix) and data (F32 / F16 arrays of that shape; BF16 uint16 bits; Q4_0 / Q8_0
    uint8 blocks [rows, K/32 * block_bytes])."""

    __slots__ = ("name", "type", "shape", "data")

    def __init__(self, name: str, ggml_type: int, shape: tuple[int, ...], data: np.ndarray):
        self.name, self.type, self.shape, self.data = name, ggml_type, tuple(shape), data

    @property
    def nbytes(self) -> int:
        return int(self.data.nbytes)

    def __repr__(self) -> str:
        return f"Tensor({self.name!r}, {type_label(self.type)}, {self.shape})"


class _Fields:
    """Sequential little-endian field reads from the mapped file, with a bounds check on each."""

    def __init__(self, mapped: np.ndarray, path: str, at: int = 0):
        self.mapped, self.path, self.at = mapped, path, at

    def take(self, dtype: np.dtype, count: int = 1) -> np.ndarray:
        end = self.at + dtype.itemsize * count
        if end > self.mapped.size:
            raise ValueError(f"{self.path}: truncated (a field ends at byte {end} of {self.mapped.size})")
        out = np.frombuffer(self.mapped, dtype=dtype, count=count, offset=self.at)
        self.at = end
        return out

    def uint(self, width: int) -> int:
        return int(self.take(np.dtype(f"<u{width}"))[0])

    def text(self) -> str:
        n = self.uint(8)
        return self.take(np.dtype("u1"), n).tobytes().decode("utf-8", errors="replace")

    def value(self, kind: int):
        if kind in _SCALAR:
            return self.take(_SCALAR[kind])[0].item()
        if kind == _STRING:
            return self.text()
        if kind == _ARRAY:
            elem, n = self.uint(4), self.uint(8)
            if elem in _SCALAR and elem != _BOOL:
                return self.take(_SCALAR[elem], n)        # numeric arrays stay numpy views
            return [self.value(elem) for _ in range(n)]
        raise ValueError(f"{self.path}: metadata value of kind {kind} is not part of the GGUF format")


class GGUF:
    """A GGUF file opened read-only: `version`, `metadata` (key -> value) and `tensors`
    (name -> Tensor).  All tensor data are views of a single read-only mapping of the file, so
    the library's bindings treat them as immutable and keep them on the device after first use."""

    def __init__(self, path: str):
        self.path = path
        self._mapped = np.memmap(path, dtype=np.uint8, mode="r")
        if self._mapped.size < 24 or self._mapped[:4].tobytes() != b"GGUF":
            raise ValueError(f"{path}: missing the GGUF magic number at the start of the file")
        f = _Fields(self._mapped, path, 4)
        self.version = f.uint(4)
        if self.version not in (2, 3):
            raise ValueError(f"{path}: format version {self.version} is not readable here (this reader handles "
                             "versions 2 and 3)")
        n_tensors, n_pairs = f.uint(8), f.uint(8)
        self.metadata: dict[str, object] = {}
        for _ in range(n_pairs):
            key = f.text()
            self.metadata[key] = f.value(f.uint(4))
        directory = []
        for _ in range(n_tensors):
            name = f.text()
            extents = [f.uint(8) for _ in range(f.uint(4))]
            directory.append((name, tuple(reversed(extents)), f.uint(4), f.uint(8)))
        align = int(self.metadata.get("general.alignment", 32))
        data_start = (f.at + align - 1) // align * align
        self.tensors: dict[str, Tensor] = {}
        for name, shape, ggml_type, offset in directory:
            self.tensors[name] = self._view(name, shape, ggml_type, data_start + offset)

    def _view(self, name: str, shape: tuple[int, ...], ggml_type: int, at: int) -> Tensor:
        if ggml_type not in GGML_TYPES:
            raise ValueError(f"{self.path}: {name} is stored as {type_label(ggml_type)}; this reader serves "
                             f"{', '.join(v[0] for v in GGML_TYPES.values())}")
        size = tensor_bytes(ggml_type, shape)
        if at + size > self._mapped.size:
            raise ValueError(f"{self.path}: {name} needs bytes {at}..{at + size} but the file has {self._mapped.size}")
        raw = self._mapped[at:at + size]
        if ggml_type in (Q4_0, Q8_0):
            row_bytes = shape[-1] // 32 * GGML_TYPES[ggml_type][1]
            data = raw.reshape(size // row_bytes, row_bytes)
        else:
            data = raw.view({F32: "<f4", F16: "<f2", BF16: "<u2"}[ggml_type]).reshape(shape)
        return Tensor(name, ggml_type, shape, data)


def dequantize_rows(t: Tensor, rows) -> np.ndarray:
    """float32 [len(rows), K] values of rows of a 2-D tensor (the embedding lookup).  A Q4_0 block
    holds d (fp16) and 16 bytes: value j is d * (low nibble of byte j - 8), value 16 + j is
    d * (high nibble of byte j - 8); a Q8_0 block holds d and 32 int8 q, value j = d * q_j."""
    idx = np.asarray(rows, dtype=np.int64).reshape(-1)
    if t.type in (F32, F16):
        return np.asarray(t.data[idx], dtype=np.float32)
    if t.type == BF16:
        return (t.data[idx].astype(np.uint32) << np.uint32(16)).view(np.float32)
    K = t.shape[-1]
    block_bytes = GGML_TYPES[t.type][1]
    blocks = np.asarray(t.data[idx]).reshape(idx.size, K // 32, block_bytes)
    scale = blocks[:, :, 0:2].copy().view("<f2").astype(np.float32)        # [rows, K/32, 1]
    q = np.empty((idx.size, K // 32, 32), np.float32)
    if t.type == Q8_0:
        q[:] = blocks[:, :, 2:].view(np.int8)
    else:
        packed = blocks[:, :, 2:]
        q[:, :, :16] = packed & 0x0F
        q[:, :, 16:] = packed >> 4
        q -= np.float32(8)
    return (scale * q).reshape(idx.size, K)


# ─── writer ──────────────────────────────────────────────────────────────────

def _pack_value(v) -> bytes:
    if isinstance(v, bool):
        return struct.pack("<I?", _BOOL, v)
    if isinstance(v, int):
        return struct.pack("<Ii", _I32, v) if -2 ** 31 <= v < 2 ** 31 else struct.pack("<Iq", _I64, v)
    if isinstance(v, float):
        return struct.pack("<If", _F32, v)
    if isinstance(v, str):
        b = v.encode()
        return struct.pack("<IQ", _STRING, len(b)) + b
    if isinstance(v, tuple) and len(v) == 2 and v[0] in ("u32", "u64", "f64"):
        kind, x = v
        if kind == "u32":
            return struct.pack("<II", _U32, x)
        if kind == "u64":
            return struct.pack("<IQ", _U64, x)
        return struct.pack("<Id", _F64, x)
    raise TypeError(f"unsupported metadata value {v!r}")


def write(path: str, metadata: dict, tensors: Iterable[tuple[str, int, tuple[int, ...], object]],
          alignment: int = 32) -> None:
    """Write a GGUF v3 file.  tensors: (name, ggml_type, shape outermost first, data) where data
    is an array of the tensor's bytes or a zero-argument callable returning it (called once, in
    order, so large tensors can be produced one at a time)."""
    tensors = list(tensors)
    md = dict(metadata)
    md["general.alignment"] = ("u32", alignment)
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(md)))
    for k, v in md.items():
        kb = k.encode()
        head += struct.pack("<Q", len(kb)) + kb + _pack_value(v)
    offset = 0
    offsets = []
    for name, ttype, shape, _ in tensors:
        nb = name.encode()
        head += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(shape))
        for d in reversed(shape):
            head += struct.pack("<Q", int(d))
        head += struct.pack("<IQ", ttype, offset)
        offsets.append(offset)
        offset += -(-tensor_bytes(ttype, shape) // alignment) * alignment
    pad = -len(head) % alignment
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(head)
        f.write(b"\0" * pad)
        for (name, ttype, shape, data), off in zip(tensors, offsets):
            arr = np.ascontiguousarray(data() if callable(data) else data)
            want = tensor_bytes(ttype, shape)
            if arr.nbytes != want:
                raise ValueError(f"{name}: {arr.nbytes} bytes, {want} expected")
            f.write(arr.view(np.uint8).reshape(-1).data)
            f.write(b"\0" * (-want % alignment))
    os.replace(tmp, path)


def write_config(model_dir: str, config: dict) -> str:
    os.makedirs(model_dir, exist_ok=True)
    path = os.path.join(model_dir, "config.json")
    with open(path, "w") as f:
        json.dump(config, f, indent=1)
    return path
