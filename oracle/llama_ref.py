"""CPU restatement of the reference's Llama decode loop.  TEST INFRASTRUCTURE ONLY.

Restates examples/llama/llama.py's GGUF path (step :414-439, _attention :398-412, generate
:481-505, rms_norm :184-187, _rope :387-396, rope_inv_freq/rope_cos_sin :131-166,
dequantize_rows gguf_reader.py:112-129) on the CPU, with the kernels taken from either

* "reference": the reference's own kernel table compiled from its sources (oracle/_ref,
  widest table this CPU runs: gemv_q4_0/gemv_q8_0, sgemm, softmax_row, silu), i.e. the
  reference's CPU path itself, or
* "simd": this oracle's C restatement of the reference's SIMD tables' arithmetic orders (the
  Q4_0 row loop of q4_0_rows.hpp, the AVX-512 few-row trans_b dot, the AVX2 direct product,
  softmax_row_avx2, silu_avx2), bit-exact with "reference" on CPUs with AVX2 or AVX-512,
* "port": this oracle's C restatement of the scalar table (scalar GEMVs, scalar trans_b
  products, float64 softmax rounded to float32, scalar SiLU),

and a float64 evaluation of the same quantized model ("f64") that pins both: tokens where the
top-2 logit margin is wide agree across all three.

The synthetic model is generated here from its seed, independently of the product's GGUF
writer: rng = default_rng(seed); the prompt ids first, then every matrix N(0, 0.02) in the
order of synthetic_order(), quantized by this oracle's quantizers; norm weights 1.0.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from . import oracle as o

F32, Q4_0, Q8_0 = 0, 2, 8


@dataclass
class Cfg:
    n_layers: int
    hidden: int
    n_heads: int
    n_kv: int
    head_dim: int
    ffn: int
    vocab: int
    eps: float
    theta: float
    rope_scaling: dict | None

    @classmethod
    def from_config(cls, c: dict) -> "Cfg":
        heads = int(c["num_attention_heads"])
        return cls(int(c["num_hidden_layers"]), int(c["hidden_size"]), heads, int(c.get("num_key_value_heads", heads)),
                   int(c.get("head_dim") or int(c["hidden_size"]) // heads), int(c["intermediate_size"]),
                   int(c["vocab_size"]), float(c["rms_norm_eps"]), float(c.get("rope_theta", 10000.0)),
                   c.get("rope_scaling"))


def synthetic_order(c: Cfg, tied: bool = True) -> list[tuple[str, tuple[int, int]]]:
    d, f, hd = c.hidden, c.ffn, c.head_dim
    order = [("token_embd", (c.vocab, d))]
    if not tied:
        order.append(("output", (c.vocab, d)))
    for i in range(c.n_layers):
        order += [(f"{i}.attn_q", (c.n_heads * hd, d)), (f"{i}.attn_k", (c.n_kv * hd, d)),
                  (f"{i}.attn_v", (c.n_kv * hd, d)), (f"{i}.attn_output", (d, c.n_heads * hd)),
                  (f"{i}.ffn_gate", (f, d)), (f"{i}.ffn_up", (f, d)), (f"{i}.ffn_down", (d, f))]
    return order


def synthetic_model(c: Cfg, seed: int, n_prompt: int, wtype: int = Q4_0) -> tuple[list[int], dict]:
    """(prompt ids, {name: quantized bytes [rows, nb*bytes] or float32 matrix})."""
    rng = np.random.default_rng(seed)
    prompt = [int(t) for t in rng.integers(0, c.vocab, n_prompt)]
    W = {}
    for name, shape in synthetic_order(c):
        w = rng.standard_normal(shape, dtype=np.float32)
        w *= np.float32(0.02)
        W[name] = w if wtype == F32 else (o.quantize_q4_0(w) if wtype == Q4_0 else o.quantize_q8_0(w))
    return prompt, W


def dequant(wtype: int, Wq: np.ndarray, n: int, k: int) -> np.ndarray:
    """float32 [n, k] values of a quantized matrix: d * (q - 8) or d * q, exact in float32."""
    if wtype == F32:
        return np.asarray(Wq, np.float32)
    d, q = (o.q4_0_split if wtype == Q4_0 else o.q8_0_split)(Wq, n, k)
    return (d.astype(np.float32)[:, :, None] * q.astype(np.float32)).reshape(n, k)


class Decoder:
    """One sequence through the restated loop.  kind: "reference", "port" or "f64"."""

    def __init__(self, c: Cfg, W: dict, wtype: int, kind: str):
        self.c, self.W, self.wtype, self.kind = c, W, wtype, kind
        if kind == "reference":
            self.R = o.ref()
            if self.R is None:
                raise RuntimeError("oracle/_ref is not built")
            self.isa = o.ISA[o.ref_best_isa()]
        self.inv_freq = o.rope_inv_freq(c.head_dim, c.theta, c.rope_scaling)
        self.ones = np.ones(c.hidden, np.float32)
        self._deq = {}

    # kernels -------------------------------------------------------------
    def gemv(self, name: str, x: np.ndarray) -> np.ndarray:
        Wq = self.W[name]
        n = Wq.shape[0]
        k = x.size
        if self.kind == "f64":
            if name not in self._deq:
                self._deq[name] = dequant(self.wtype, Wq, n, k).astype(np.float64)
            return self._deq[name] @ x.astype(np.float64)
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(n, np.float32)
        if self.wtype == F32:
            return self.sgemm_tb(x.reshape(1, -1), Wq, 1.0)[0]
        if self.kind == "simd" and self.wtype == Q4_0:
            return o.gemv_q4_0_simd(x, Wq, n, k)
        if self.kind == "reference":
            f = self.R.ref_gemv_q4_0 if self.wtype == Q4_0 else self.R.ref_gemv_q8_0
            f(self.isa, n, k, x.ctypes.data_as(o._f32p), np.ascontiguousarray(Wq).ctypes.data_as(o._u8p),
              y.ctypes.data_as(o._f32p))
            return y
        return (o.gemv_q4_0 if self.wtype == Q4_0 else o.gemv_q8_0)(x, Wq, n, k)

    def sgemm_tb(self, A: np.ndarray, B: np.ndarray, alpha: float) -> np.ndarray:
        """alpha * A @ B.T (A [M, K], B [N, K]), as sk.sgemm(A, B, alpha=alpha, trans_b=True)."""
        A = np.ascontiguousarray(A, np.float32)
        B = np.ascontiguousarray(B, np.float32)
        M, K = A.shape
        N = B.shape[0]
        if self.kind == "reference":
            C = np.zeros((M, N), np.float32)
            self.R.ref_sgemm(self.isa, 0, 1, M, N, K, alpha, A.ctypes.data, K, B.ctypes.data, K, 0.0,
                             C.ctypes.data_as(o._f32p), N)
            return C
        if self.kind == "simd":
            return o.sgemm_tb_simd(A, B, alpha)
        return o.gemm_tb("fp32", A, B, alpha=alpha)

    def sgemm_nn(self, A: np.ndarray, B: np.ndarray) -> np.ndarray:
        """A @ B (A [M, K], B [K, N]), as sk.sgemm(A, B)."""
        A = np.ascontiguousarray(A, np.float32)
        B = np.ascontiguousarray(B, np.float32)
        M, K = A.shape
        N = B.shape[1]
        if self.kind == "reference":
            C = np.zeros((M, N), np.float32)
            self.R.ref_sgemm(self.isa, 0, 0, M, N, K, 1.0, A.ctypes.data, K, B.ctypes.data, N, 0.0,
                             C.ctypes.data_as(o._f32p), N)
            return C
        if self.kind == "simd":
            return o.sgemm_nn_simd(A, B)
        return o.gemm_tb("fp32", A, np.ascontiguousarray(B.T))

    def softmax(self, s: np.ndarray) -> np.ndarray:
        if self.kind == "reference":
            out = np.empty_like(s)
            for r in range(s.shape[0]):
                row = np.ascontiguousarray(s[r])
                orow = np.empty_like(row)
                self.R.ref_softmax_row(self.isa, row.ctypes.data_as(o._f32p), orow.ctypes.data_as(o._f32p), row.size)
                out[r] = orow
            return out
        if self.kind == "simd":
            return o.softmax_simd(s)
        return o.softmax64(s).astype(np.float32)

    def silu(self, x: np.ndarray) -> np.ndarray:
        if self.kind == "reference":
            x = np.ascontiguousarray(x, np.float32)
            y = np.empty_like(x)
            self.R.ref_silu(self.isa, x.ctypes.data_as(o._f32p), y.ctypes.data_as(o._f32p), x.size)
            return y
        if self.kind == "simd":
            return o.silu_simd(x)
        return o.silu_scalar(x)

    # the loop --------------------------------------------------------------
    def reset(self, capacity: int) -> None:
        c = self.c
        dt = np.float64 if self.kind == "f64" else np.float32
        self.kc = np.zeros((c.n_layers, c.n_kv, capacity, c.head_dim), dt)
        self.vc = np.zeros_like(self.kc)
        self.pos = 0

    def embed(self, tok: int) -> np.ndarray:
        E = self.W["token_embd"]
        row = dequant(self.wtype, E[tok:tok + 1], 1, self.c.hidden)[0]
        return row.astype(np.float64) if self.kind == "f64" else row

    def step(self, tok: int) -> np.ndarray:
        c = self.c
        nh, nkv, hd = c.n_heads, c.n_kv, c.head_dim
        pos = self.pos
        f64 = self.kind == "f64"
        cos, sin = o.rope_cos_sin(self.inv_freq, pos)
        x = self.embed(tok)
        for i in range(c.n_layers):
            h = o.rms_norm64(x, self.ones, c.eps) if f64 else o.rms_norm(x, self.ones, c.eps)
            q = self.gemv(f"{i}.attn_q", h).reshape(nh, hd)
            k = self.gemv(f"{i}.attn_k", h).reshape(nkv, hd)
            v = self.gemv(f"{i}.attn_v", h).reshape(nkv, hd)
            if f64:
                q, k = _rope64(q, cos, sin), _rope64(k, cos, sin)
            else:
                q, k = o.rope(q, cos, sin, True), o.rope(k, cos, sin, True)
            x = x + self.gemv(f"{i}.attn_output", self.attention(i, q, k, v, pos))
            h = o.rms_norm64(x, self.ones, c.eps) if f64 else o.rms_norm(x, self.ones, c.eps)
            g, u = self.gemv(f"{i}.ffn_gate", h), self.gemv(f"{i}.ffn_up", h)
            m = (g / (1.0 + np.exp(-g))) * u if f64 else self.silu(g) * u
            x = x + self.gemv(f"{i}.ffn_down", m)
        self.pos = pos + 1
        h = o.rms_norm64(x, self.ones, c.eps) if f64 else o.rms_norm(x, self.ones, c.eps)
        return self.gemv("token_embd", h)

    def attention(self, li: int, q, k, v, pos: int):
        c = self.c
        nh, nkv, hd = c.n_heads, c.n_kv, c.head_dim
        rep = nh // nkv
        self.kc[li][:, pos] = k
        self.vc[li][:, pos] = v
        scale = 1.0 / math.sqrt(hd)
        out = np.empty((nh, hd), self.kc.dtype)
        for g in range(nkv):
            qg = q[g * rep:(g + 1) * rep]
            K, V = self.kc[li][g, :pos + 1], self.vc[li][g, :pos + 1]
            if self.kind == "f64":
                s = scale * (qg @ K.T)
                e = np.exp(s - s.max(axis=1, keepdims=True))
                out[g * rep:(g + 1) * rep] = (e / e.sum(axis=1, keepdims=True)) @ V
            else:
                s = self.sgemm_tb(qg, K, scale)
                out[g * rep:(g + 1) * rep] = self.sgemm_nn(self.softmax(s), V)
        return out.reshape(-1)

    def generate(self, prompt: list[int], n_new: int) -> tuple[list[int], list[float], np.ndarray]:
        """Greedy ids, the top-2 logit margin of each, and the last logits (stop_at_eos=False)."""
        self.reset(len(prompt) + n_new)
        logits = None
        for t in prompt:
            logits = self.step(t)
        ids, margins = [], []
        for i in range(n_new):
            nxt = int(np.argmax(logits))
            top2 = np.partition(np.asarray(logits, np.float64), -2)[-2:]
            ids.append(nxt)
            margins.append(float(top2[1] - top2[0]))
            if i == n_new - 1:
                break
            logits = self.step(nxt)
        return ids, margins, np.asarray(logits)


def _rope64(x, cos, sin):
    half = x.shape[-1] // 2
    a, b = x[:, 0::2], x[:, 1::2]
    c, s = cos[:half].astype(np.float64), sin[:half].astype(np.float64)
    out = np.empty_like(x)
    out[:, 0::2] = a * c - b * s
    out[:, 1::2] = b * c + a * s
    return out
