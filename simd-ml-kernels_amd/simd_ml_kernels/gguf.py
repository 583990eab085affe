"""GGUF files (llama.cpp's model format, versions 2 and 3): a memory-mapped reader that returns
every tensor as a numpy view (no copy), and a writer for the synthetic models of the decode
benchmark.

The reader covers what examples/llama/gguf_reader.py:39-129 reads: metadata of every GGUF value
type, and F32 / F16 / BF16 / Q8_0 / Q4_0 tensors.  Quantized tensors come back as their raw
uint8 blocks [rows, K/32 * block_bytes] -- the bytes gemv_q4_0 / gemv_q8_0 take.  Layout:
"GGUF", u32 version, u64 tensor count, u64 metadata count; metadata entries (string key, u32
type, value); tensor infos (string name, u32 n_dims, u64 dims innermost first, u32 ggml type,
u64 offset); tensor data from the next multiple of general.alignment (32 by default).
"""

from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass
from typing import Iterable

import numpy as np

F32, F16, Q4_0, Q8_0, BF16 = 0, 1, 2, 8, 30
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", BF16: "BF16"}
# (bytes per block, values per block)
BLOCK = {F32: (4, 1), F16: (2, 1), BF16: (2, 1), Q4_0: (18, 32), Q8_0: (34, 32)}

# GGUF metadata value types.
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_FMT = {_U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f", _BOOL: "<?",
        _U64: "<Q", _I64: "<q", _F64: "<d"}


@dataclass
class Tensor:
    name: str
    type: int
    shape: tuple[int, ...]  # outermost first: [N, K] for a weight matrix
    data: np.ndarray        # F32/F16: that dtype and shape; BF16: uint16; Q4_0/Q8_0: uint8 [rows, K/32*bytes]

    @property
    def type_name(self) -> str:
        return TYPE_NAMES.get(self.type, str(self.type))

    @property
    def nbytes(self) -> int:
        return int(self.data.nbytes)


def tensor_bytes(ggml_type: int, shape: Iterable[int]) -> int:
    shape = tuple(int(s) for s in shape)
    bsize, bvals = BLOCK[ggml_type]
    k = shape[-1]
    rows = int(np.prod(shape[:-1], dtype=np.int64)) if len(shape) > 1 else 1
    if k % bvals:
        raise ValueError(f"row length {k} is not a multiple of {bvals}")
    return rows * (k // bvals) * bsize


class _Cursor:
    def __init__(self, buf: np.ndarray, path: str):
        self.buf, self.pos, self.path = buf, 0, path

    def scalar(self, fmt: str):
        (v,) = struct.unpack_from(fmt, self.buf, self.pos)
        self.pos += struct.calcsize(fmt)
        return v

    def string(self) -> str:
        n = self.scalar("<Q")
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8", errors="replace")
        self.pos += n
        return s

    def value(self, vtype: int):
        if vtype in _FMT:
            return self.scalar(_FMT[vtype])
        if vtype == _STR:
            return self.string()
        if vtype == _ARR:
            etype, n = self.scalar("<I"), self.scalar("<Q")
            if etype in _FMT and etype != _BOOL:
                dt = np.dtype(_FMT[etype])
                a = np.frombuffer(self.buf, dtype=dt, count=n, offset=self.pos)
                self.pos += n * dt.itemsize
                return a
            return [self.value(etype) for _ in range(n)]
        raise ValueError(f"{self.path}: unknown GGUF metadata type {vtype}")


class GGUF:
    """A GGUF file opened read-only: .version, .metadata (dict), .tensors (name -> Tensor).
    Tensor data are views of one read-only memory map, so the library keeps them device-resident
    after their first use (read-only all the way down)."""

    def __init__(self, path: str):
        self.path = path
        mm = np.memmap(path, dtype=np.uint8, mode="r")
        self._mm = mm
        if mm.size < 24 or bytes(mm[:4]) != b"GGUF":
            raise ValueError(f"{path}: not a GGUF file")
        cur = _Cursor(mm, path)
        cur.pos = 4
        self.version = cur.scalar("<I")
        if self.version not in (2, 3):
            raise ValueError(f"{path}: GGUF version {self.version} (2 and 3 are supported)")
        n_tensors, n_kv = cur.scalar("<Q"), cur.scalar("<Q")
        self.metadata: dict[str, object] = {}
        for _ in range(n_kv):
            key = cur.string()
            self.metadata[key] = cur.value(cur.scalar("<I"))
        infos = []
        for _ in range(n_tensors):
            name = cur.string()
            n_dims = cur.scalar("<I")
            dims = [cur.scalar("<Q") for _ in range(n_dims)]
            infos.append((name, dims, cur.scalar("<I"), cur.scalar("<Q")))
        align = int(self.metadata.get("general.alignment", 32))
        base = -(-cur.pos // align) * align
        self.tensors: dict[str, Tensor] = {}
        for name, dims, ttype, offset in infos:
            if ttype not in BLOCK:
                raise ValueError(f"{path}: tensor {name} has ggml type {ttype} (F32, F16, BF16, Q8_0 or Q4_0 expected)")
            shape = tuple(int(d) for d in reversed(dims))
            nbytes = tensor_bytes(ttype, shape)
            start = base + offset
            if start + nbytes > mm.size:
                raise ValueError(f"{path}: tensor {name} runs past the end of the file")
            raw = mm[start:start + nbytes]
            if ttype == F32:
                data = raw.view("<f4").reshape(shape)
            elif ttype in (F16,):
                data = raw.view("<f2").reshape(shape)
            elif ttype == BF16:
                data = raw.view("<u2").reshape(shape)
            else:
                rows = nbytes // (shape[-1] // 32 * BLOCK[ttype][0])
                data = raw.reshape(rows, nbytes // rows)
            self.tensors[name] = Tensor(name, ttype, shape, data)


def dequantize_rows(t: Tensor, rows) -> np.ndarray:
    """float32 values of rows of a 2-D tensor (the embedding lookup): d * (q - 8) for Q4_0 (value j
    in the low nibble of byte j, value 16 + j in the high nibble), d * q for Q8_0."""
    r = np.atleast_1d(np.asarray(rows, dtype=np.int64))
    if t.type == F32:
        return np.array(t.data[r], dtype=np.float32)
    if t.type == F16:
        return t.data[r].astype(np.float32)
    if t.type == BF16:
        return (t.data[r].astype(np.uint32) << 16).view(np.float32)
    k = t.shape[-1]
    bsize = BLOCK[t.type][0]
    blk = np.asarray(t.data[r]).reshape(len(r), k // 32, bsize)
    d = np.ascontiguousarray(blk[:, :, :2]).view("<f2").astype(np.float32)  # [rows, nb, 1]
    if t.type == Q8_0:
        q = blk[:, :, 2:].view(np.int8).astype(np.float32)
    else:
        nib = blk[:, :, 2:]
        q = np.concatenate([nib & 0x0F, nib >> 4], axis=2).astype(np.float32) - np.float32(8)
    return (d * q).reshape(len(r), k)


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
        return struct.pack("<IQ", _STR, len(b)) + b
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
