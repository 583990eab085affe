"""Llama-3.x greedy decode on the MI355X from a GGUF file.

The interface of the reference's example model (examples/llama/llama.py: Config, Llama with
reset / step / generate / weight_bytes, rope_inv_freq, rope_cos_sin) on two execution paths:

* ``device_loop=True`` (default): the whole per-token step runs on the GPU through the
  library's decode engine (smk_llama_* in include/smk_hip.h): weights uploaded once, KV cache
  in HBM, [q|k|v] and [gate|up] as one GEMV each, residual adds fused into the GEMV epilogue,
  one HIP graph per token and the greedy argmax on the device.
* ``device_loop=False``: the example's own loop (llama.py:414-439), one library call per
  operation from numpy -- gemv_q4_0 / gemv_q8_0 / sgemm for every projection, rms_norm and
  rope on the device, sgemm + softmax per KV head for attention.  This is what the
  reference's unchanged example does with this module underneath.

Both paths compute the same arithmetic: RMSNorm and RoPE bit-exact with the example's numpy
formulas, the GEMVs to the reference's error bound.  RoPE tables come from numpy on the host,
as in the example (llama.py:162-166).
"""

from __future__ import annotations

import json
import math
import os
import time
from dataclasses import dataclass, field
from typing import Iterator, Sequence

import numpy as np

from . import _core as sk
from . import abi
from . import gguf as ggufmod

# ─── configuration ───────────────────────────────────────────────────────────


@dataclass
class Config:
    """The config.json fields the decode loop uses (llama.py:73-123)."""
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    vocab_size: int
    rms_norm_eps: float
    rope_theta: float
    rope_scaling: dict | None
    tie_word_embeddings: bool
    bos_token_id: int | None = None
    eos_token_ids: tuple[int, ...] = field(default_factory=tuple)

    @classmethod
    def from_dict(cls, c: dict, generation: dict | None = None) -> "Config":
        reason = _unsupported_architecture(c)
        if reason:
            raise ValueError(f"this decode engine runs Llama models only: {reason}")
        eos = (generation or {}).get("eos_token_id", c.get("eos_token_id"))
        eos_ids = tuple(eos) if isinstance(eos, list) else (() if eos is None else (int(eos),))
        heads = int(c["num_attention_heads"])
        return cls(hidden_size=int(c["hidden_size"]), intermediate_size=int(c["intermediate_size"]),
                   num_hidden_layers=int(c["num_hidden_layers"]), num_attention_heads=heads,
                   num_key_value_heads=int(c.get("num_key_value_heads", heads)),
                   head_dim=int(c.get("head_dim") or int(c["hidden_size"]) // heads),
                   vocab_size=int(c["vocab_size"]), rms_norm_eps=float(c["rms_norm_eps"]),
                   rope_theta=float(c.get("rope_theta", 10000.0)), rope_scaling=c.get("rope_scaling"),
                   tie_word_embeddings=bool(c.get("tie_word_embeddings", False)),
                   bos_token_id=c.get("bos_token_id"), eos_token_ids=eos_ids)

    @classmethod
    def from_dir(cls, model_dir: str) -> "Config":
        with open(os.path.join(model_dir, "config.json")) as f:
            c = json.load(f)
        gen_path = os.path.join(model_dir, "generation_config.json")
        gen = None
        if os.path.exists(gen_path):
            with open(gen_path) as f:
                gen = json.load(f)
        return cls.from_dict(c, gen)


def _unsupported_architecture(c: dict) -> str | None:
    """Why a config.json describes a model the engine cannot run (None when it can): it must be
    model_type "llama" with SiLU gating and no bias terms (the example's model, llama.py:73-123)."""
    checks = (("model_type", c.get("model_type") == "llama", "model_type is {!r}"),
              ("attention_bias", not c.get("attention_bias"), "attention_bias is {!r}"),
              ("mlp_bias", not c.get("mlp_bias"), "mlp_bias is {!r}"),
              ("hidden_act", c.get("hidden_act", "silu") == "silu", "hidden_act is {!r}"))
    for key, ok, text in checks:
        if not ok:
            return text.format(c.get(key))
    return None


# Llama-3.2-1B's architecture: the shape of the synthetic benchmark model.
LLAMA_3_2_1B = {
    "model_type": "llama", "hidden_size": 2048, "intermediate_size": 8192, "num_hidden_layers": 16,
    "num_attention_heads": 32, "num_key_value_heads": 8, "head_dim": 64, "vocab_size": 128256,
    "rms_norm_eps": 1e-5, "rope_theta": 500000.0, "tie_word_embeddings": True, "hidden_act": "silu",
    "rope_scaling": {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                     "original_max_position_embeddings": 8192},
    "bos_token_id": 128000, "eos_token_id": 128001, "max_position_embeddings": 131072,
}

# ─── RoPE (numpy on the host, as the example) ────────────────────────────────


def rope_inv_freq(cfg: Config) -> np.ndarray:
    """Inverse frequencies in float32, transformers' default and llama3 rules (llama.py:131-159):
    theta^(-2i/d); with llama3 scaling, wavelengths above original/low_freq_factor are divided by
    `factor`, those below original/high_freq_factor kept, and the band between interpolated."""
    d = cfg.head_dim
    expo = np.arange(0, d, 2, dtype=np.int64).astype(np.float32) / np.float32(d)
    base = (np.float32(1.0) / (np.float32(cfg.rope_theta) ** expo)).astype(np.float32)
    rs = cfg.rope_scaling
    kind = None if rs is None else rs.get("rope_type", rs.get("type"))
    if kind in (None, "default"):
        return base
    if kind != "llama3":
        raise ValueError(f"rope_scaling type {kind!r} is not implemented (llama3 and default are)")
    factor = rs["factor"]
    lo_f, hi_f = rs["low_freq_factor"], rs["high_freq_factor"]
    orig = rs["original_max_position_embeddings"]
    wavelen = (np.float32(2 * math.pi) / base).astype(np.float32)
    long_wl, short_wl = orig / lo_f, orig / hi_f
    scaled = np.where(wavelen > long_wl, base / np.float32(factor), base).astype(np.float32)
    t = ((np.float32(orig) / wavelen - np.float32(lo_f)) / np.float32(hi_f - lo_f)).astype(np.float32)
    blended = ((1 - t) * scaled / np.float32(factor) + t * scaled).astype(np.float32)
    band = ~(wavelen < short_wl) & ~(wavelen > long_wl)
    return np.where(band, blended, scaled).astype(np.float32)


def rope_cos_sin(inv_freq: np.ndarray, pos: int) -> tuple[np.ndarray, np.ndarray]:
    """cos and sin of one position, [head_dim] with the two halves equal (llama.py:162-166)."""
    ang = (np.float32(pos) * inv_freq).astype(np.float32)
    both = np.concatenate([ang, ang])
    return np.cos(both), np.sin(both)


def rope_tables(inv_freq: np.ndarray, capacity: int) -> tuple[np.ndarray, np.ndarray]:
    """[capacity, head_dim] cos and sin, each row exactly rope_cos_sin(inv_freq, pos)."""
    rows = [rope_cos_sin(inv_freq, p) for p in range(capacity)]
    return (np.ascontiguousarray(np.stack([r[0] for r in rows]), dtype=np.float32),
            np.ascontiguousarray(np.stack([r[1] for r in rows]), dtype=np.float32))


# ─── model ──────────────────────────────────────────────────────────────────

_LAYER_TENSORS = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm", "ffn_gate", "ffn_up",
                  "ffn_down")
_MATRIX_TYPES = {ggufmod.F32: "f32", ggufmod.Q8_0: "q8_0", ggufmod.Q4_0: "q4_0"}
SECTIONS = ("gemv", "attention", "norm_rope_silu")


class _Linear:
    """y = x @ W.T for one row x through the module (the example's Linear, llama.py:190-211)."""

    def __init__(self, t: ggufmod.Tensor):
        if t.type not in _MATRIX_TYPES:
            raise ValueError(f"{t.name} is {ggufmod.type_label(t.type)}; F32, Q8_0 or Q4_0 expected")
        self.kind, self.data, self.shape = _MATRIX_TYPES[t.type], t.data, t.shape
        n, k = t.shape
        if self.kind == "q4_0":
            self._f = lambda x: sk.gemv_q4_0(x, self.data, n, k)
        elif self.kind == "q8_0":
            self._f = lambda x: sk.gemv_q8_0(x, self.data, n, k)
        else:
            self._f = lambda x: sk.sgemm(x.reshape(1, -1), self.data, trans_b=True)[0]

    def __call__(self, x: np.ndarray) -> np.ndarray:
        return self._f(x)

    @property
    def nbytes(self) -> int:
        return int(self.data.nbytes)


class Llama:
    """Llama-3.x decoder for one sequence, from a GGUF file (F32 / Q8_0 / Q4_0 matrices, F32
    norms, tied or separate output matrix).  config.json comes from model_dir; when model_dir is
    None the GGUF's own llama.* metadata gives the configuration."""

    def __init__(self, model_dir: str | None = None, weights: str = "fp32", gguf: str | None = None, *,
                 device_loop: bool = True):
        path = gguf
        if path is None:
            if weights == "fp32":
                raise NotImplementedError("safetensors checkpoints are not read by this build; pass gguf=<file>")
            if model_dir is None:
                raise ValueError("a GGUF file is required (gguf=...)")
            path = find_gguf(model_dir, weights)
        self.gguf = g = ggufmod.GGUF(path)
        self.cfg = cfg = Config.from_dir(model_dir) if model_dir is not None else config_from_gguf(g)
        _check_metadata(g, cfg, path)
        self.device_loop = device_loop
        self.rope_interleaved = True  # GGUF q/k rows are in Meta's order: pairs (2i, 2i+1)
        self.inv_freq = rope_inv_freq(cfg)
        T = g.tensors
        used = {"token_embd.weight", "output_norm.weight"}
        self._emb = T["token_embd.weight"]
        self._head_name = "output.weight" if "output.weight" in T else "token_embd.weight"
        used.add(self._head_name)
        for i in range(cfg.num_hidden_layers):
            used.update(f"blk.{i}.{n}.weight" for n in _LAYER_TENSORS)
        leftover = sorted(set(T) - used - {"rope_freqs.weight"})
        if leftover:
            raise KeyError(f"{path}: unused tensors {leftover[:5]}")
        self._check_shapes()
        types: dict[str, int] = {}
        for t in T.values():
            label = ggufmod.type_label(t.type)
            types[label] = types.get(label, 0) + 1
        self.weight_types = types
        self.k_cache: np.ndarray | None = None
        self.v_cache: np.ndarray | None = None
        self.pos = 0
        self.capacity = 0
        self.last_logits: np.ndarray | None = None
        self.profile: dict[str, float] | None = None
        self._engine = None
        if device_loop:
            self._engine = _Engine(self)
        else:
            self._host_setup()

    # -- loading ------------------------------------------------------------

    def _tensor(self, name: str) -> ggufmod.Tensor:
        return self.gguf.tensors[name]

    def _check_shapes(self) -> None:
        c = self.cfg
        d, f, hd = c.hidden_size, c.intermediate_size, c.head_dim
        want = {"attn_q": (c.num_attention_heads * hd, d), "attn_k": (c.num_key_value_heads * hd, d),
                "attn_v": (c.num_key_value_heads * hd, d), "attn_output": (d, c.num_attention_heads * hd),
                "ffn_gate": (f, d), "ffn_up": (f, d), "ffn_down": (d, f), "attn_norm": (d,), "ffn_norm": (d,)}
        for i in range(c.num_hidden_layers):
            for name, shape in want.items():
                t = self._tensor(f"blk.{i}.{name}.weight")
                if tuple(t.shape) != shape:
                    raise ValueError(f"blk.{i}.{name}: shape {t.shape}, config says {shape}")
        for name in ("token_embd.weight", self._head_name):
            if tuple(self._tensor(name).shape) != (c.vocab_size, d):
                raise ValueError(f"{name}: shape does not match the config")
        if tuple(self._tensor("output_norm.weight").shape) != (d,):
            raise ValueError("output_norm: shape does not match the config")

    def _host_setup(self) -> None:
        c = self.cfg
        self._lin = {}
        for i in range(c.num_hidden_layers):
            for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"):
                self._lin[(i, n)] = _Linear(self._tensor(f"blk.{i}.{n}.weight"))
        self._lm_head = _Linear(self._tensor(self._head_name))
        self._norms = {(i, n): np.asarray(self._tensor(f"blk.{i}.{n}.weight").data, np.float32)
                       for i in range(c.num_hidden_layers) for n in ("attn_norm", "ffn_norm")}
        self._out_norm = np.asarray(self._tensor("output_norm.weight").data, np.float32)

    def weight_bytes(self) -> int:
        """Bytes of the weight matrices one token reads (every projection and the lm_head once)."""
        c = self.cfg
        total = self._tensor(self._head_name).nbytes
        for i in range(c.num_hidden_layers):
            for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"):
                total += self._tensor(f"blk.{i}.{n}.weight").nbytes
        return total

    # -- decoding ------------------------------------------------------------

    def reset(self, capacity: int) -> None:
        """Empty KV cache for up to `capacity` positions."""
        c = self.cfg
        self.capacity = capacity
        self.pos = 0
        if self._engine is not None:
            self._engine.reset(capacity)
        else:
            shape = (c.num_hidden_layers, c.num_key_value_heads, capacity, c.head_dim)
            self.k_cache = np.zeros(shape, np.float32)
            self.v_cache = np.zeros(shape, np.float32)

    def step(self, token: int, logits: bool = True) -> np.ndarray | None:
        """Run one token at position self.pos; float32 logits [vocab] (None with logits=False)."""
        if self.capacity == 0:
            raise RuntimeError("call reset() first")
        if self.pos >= self.capacity:
            raise ValueError(f"KV cache full ({self.capacity} positions)")
        if self._engine is not None and self.profile is not None:
            out = self._engine.step_profile(int(token), logits, self.profile)
        elif self._engine is not None:
            out = self._engine.step(int(token), logits)
        elif self.profile is not None:
            out = self._host_step(int(token), logits, self.profile)
        else:
            out = self._host_step(int(token), logits, None)
        self.pos += 1
        if out is not None:
            self.last_logits = out
        return out

    def _host_step(self, token: int, want_logits: bool, prof: dict | None) -> np.ndarray | None:
        """The example's step (llama.py:414-439) with one module call per operation."""
        c = self.cfg
        nh, nkv, hd, eps = c.num_attention_heads, c.num_key_value_heads, c.head_dim, c.rms_norm_eps
        pos = self.pos
        clock = time.perf_counter
        acc = {"gemv": 0.0, "attention": 0.0, "norm_rope_silu": 0.0}
        t_all = clock()

        def timed(section, f, *a):
            if prof is None:
                return f(*a)
            t = clock()
            r = f(*a)
            acc[section] += clock() - t
            return r

        cos, sin = rope_cos_sin(self.inv_freq, pos)
        x = ggufmod.dequantize_rows(self._emb, token)[0]
        for i in range(c.num_hidden_layers):
            lin = lambda n: self._lin[(i, n)]
            h = timed("norm_rope_silu", sk.rms_norm, x, self._norms[(i, "attn_norm")], eps)
            q = timed("gemv", lin("attn_q"), h)
            k = timed("gemv", lin("attn_k"), h)
            v = timed("gemv", lin("attn_v"), h)
            q = timed("norm_rope_silu", sk.rope, q.reshape(nh, hd), cos, sin, True)
            k = timed("norm_rope_silu", sk.rope, k.reshape(nkv, hd), cos, sin, True)
            a = timed("attention", self._host_attention, i, q, k, v.reshape(nkv, hd), pos)
            x = x + timed("gemv", lin("attn_output"), a)
            h = timed("norm_rope_silu", sk.rms_norm, x, self._norms[(i, "ffn_norm")], eps)
            gate = timed("gemv", lin("ffn_gate"), h)
            up = timed("gemv", lin("ffn_up"), h)
            m = timed("norm_rope_silu", lambda g, u: sk.silu(g) * u, gate, up)
            x = x + timed("gemv", lin("ffn_down"), m)
        out = None
        if want_logits:
            h = timed("norm_rope_silu", sk.rms_norm, x, self._out_norm, eps)
            out = timed("gemv", self._lm_head, h)
        if prof is not None:
            for k_, v_ in acc.items():
                prof[k_] = prof.get(k_, 0.0) + v_
            prof["total"] = prof.get("total", 0.0) + clock() - t_all
            prof["steps"] = prof.get("steps", 0) + 1
        return out

    def _host_attention(self, li: int, q: np.ndarray, k: np.ndarray, v: np.ndarray, pos: int) -> np.ndarray:
        """Cache write, then per KV head: scores = scale q K^T, softmax, p V (llama.py:398-412)."""
        c = self.cfg
        nh, nkv, hd = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        rep = nh // nkv
        kc, vc = self.k_cache[li], self.v_cache[li]
        kc[:, pos] = k
        vc[:, pos] = v
        out = np.empty((nh, hd), np.float32)
        scale = 1.0 / math.sqrt(hd)
        for g in range(nkv):
            qg = np.ascontiguousarray(q[g * rep:(g + 1) * rep])
            s = sk.sgemm(qg, kc[g, :pos + 1], alpha=scale, trans_b=True)
            out[g * rep:(g + 1) * rep] = sk.sgemm(sk.softmax(s), vc[g, :pos + 1])
        return out.reshape(-1)

    def generate(self, prompt_ids: Sequence[int], max_new_tokens: int, stats: dict | None = None,
                 stop_at_eos: bool = True) -> Iterator[int]:
        """Greedy decode (llama.py:481-505): prefill the prompt, then yield up to max_new_tokens
        ids, stopping after an EOS id unless stop_at_eos is False.  On the device path the whole
        run is one engine call (argmax on the GPU, tokens copied back at the end): tokens after an
        EOS never change those before it, so stopping is a truncation.  The device path prefills
        quantized models in chunks of prompt rows (set_prefill_rows), the reference's loop one
        token at a time; the cache and the tokens are the same bit for bit."""
        prompt = [int(t) for t in prompt_ids]
        if max_new_tokens <= 0:
            return
        self.reset(len(prompt) + max_new_tokens)
        if self._engine is not None:
            ids, pre_s, dec_s = self._engine.generate(prompt, max_new_tokens)
            self.pos = len(prompt) + max_new_tokens - 1
            if stats is not None:
                stats.update(prefill_s=pre_s, prefill_tokens=len(prompt), decode_s=dec_s,
                             decode_steps=max_new_tokens - 1)
            for nxt in ids:
                yield int(nxt)
                if stop_at_eos and nxt in self.cfg.eos_token_ids:
                    return
            return
        t0 = time.perf_counter()
        logits = None
        for tok in prompt:
            logits = self.step(tok)
        if stats is not None:
            stats.update(prefill_s=time.perf_counter() - t0, prefill_tokens=len(prompt), decode_s=0.0,
                         decode_steps=0)
        for i in range(max_new_tokens):
            nxt = int(np.argmax(logits))
            yield nxt
            if (stop_at_eos and nxt in self.cfg.eos_token_ids) or i == max_new_tokens - 1:
                break
            t = time.perf_counter()
            logits = self.step(nxt)
            if stats is not None:
                stats["decode_s"] += time.perf_counter() - t
                stats["decode_steps"] += 1

    def set_prefill_rows(self, rows: int) -> None:
        """Device path: prompt rows per prefill chunk (0 or 1: one decode step per prompt token)."""
        if self._engine is not None:
            self._engine.set_prefill_rows(int(rows))

    def close(self) -> None:
        if self._engine is not None:
            self._engine.close()
            self._engine = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _Engine:
    """The device decode engine (smk_llama_*): weights uploaded once at construction."""

    def __init__(self, model: Llama):
        c = model.cfg
        g = model.gguf
        L = abi.lib()
        self.L = L
        emb = g.tensors["token_embd.weight"]
        head = g.tensors.get("output.weight")
        mtypes = {g.tensors[f"blk.{i}.{n}.weight"].type for i in range(c.num_hidden_layers)
                  for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")}
        if len(mtypes) != 1:
            raise ValueError(f"the device loop needs one type for every layer matrix (found {sorted(mtypes)})")
        cfgs = abi.LlamaConfig(n_layers=c.num_hidden_layers, hidden=c.hidden_size, n_heads=c.num_attention_heads,
                               n_kv_heads=c.num_key_value_heads, head_dim=c.head_dim, ffn=c.intermediate_size,
                               vocab=c.vocab_size, matrix_type=mtypes.pop(), embed_type=emb.type,
                               head_type=-1 if head is None else head.type, rope_interleaved=1,
                               rms_eps=c.rms_norm_eps)
        h = abi.ctypes.c_void_p()
        abi.check(L.smk_llama_create(abi.ctypes.byref(cfgs), abi.ctypes.byref(h)), "smk_llama_create")
        self.h = h
        self.cfg = c
        self.inv_freq = model.inv_freq
        ids = abi.LLAMA_TENSORS

        def put(tid: int, layer: int, t: ggufmod.Tensor):
            a = np.ascontiguousarray(t.data)
            abi.check(L.smk_llama_set_tensor(self.h, tid, layer, a.ctypes.data, a.nbytes), f"load {t.name}")

        put(ids["token_embd"], 0, emb)
        put(ids["output_norm"], 0, g.tensors["output_norm.weight"])
        if head is not None:
            put(ids["output"], 0, head)
        for i in range(c.num_hidden_layers):
            for n in _LAYER_TENSORS:
                put(ids[n], i, g.tensors[f"blk.{i}.{n}.weight"])
        self.logits = np.empty(c.vocab_size, np.float32)

    def reset(self, capacity: int) -> None:
        cos, sin = rope_tables(self.inv_freq, capacity)
        abi.check(self.L.smk_llama_reset(self.h, capacity, cos.ctypes.data, sin.ctypes.data), "smk_llama_reset")

    def step(self, token: int, logits: bool) -> np.ndarray | None:
        out = np.empty(self.cfg.vocab_size, np.float32) if logits else None
        abi.check(self.L.smk_llama_step(self.h, token, out.ctypes.data if logits else None), "smk_llama_step")
        return out

    DEVICE_SECTIONS = ("embed", "rms_norm", "gemv_qkv", "rope_kv", "attention", "gemv_o", "gemv_gate_up",
                       "silu_mul", "gemv_down", "lm_head", "argmax")
    # The example's profile sections (llama.py:441-479) from the device sections.
    _GROUPS = {"gemv": ("gemv_qkv", "gemv_o", "gemv_gate_up", "gemv_down", "lm_head"), "attention": ("attention",),
               "norm_rope_silu": ("rms_norm", "rope_kv", "silu_mul")}

    def step_profile(self, token: int, logits: bool, prof: dict) -> np.ndarray | None:
        """One eager step with a HIP event per section; seconds summed into prof like the example's
        profile dict (gemv, attention, norm_rope_silu, total, steps), device sections in
        prof["device"]."""
        out = np.empty(self.cfg.vocab_size, np.float32) if logits else None
        ms = np.zeros(len(self.DEVICE_SECTIONS), np.float64)
        abi.check(self.L.smk_llama_step_profile(self.h, token, out.ctypes.data if logits else None, ms.ctypes.data,
                                                len(ms)), "smk_llama_step_profile")
        dev = prof.setdefault("device", {})
        for name, v in zip(self.DEVICE_SECTIONS, ms):
            dev[name] = dev.get(name, 0.0) + v * 1e-3
        for grp, names in self._GROUPS.items():
            prof[grp] = prof.get(grp, 0.0) + sum(ms[self.DEVICE_SECTIONS.index(n)] for n in names) * 1e-3
        prof["total"] = prof.get("total", 0.0) + float(ms.sum()) * 1e-3
        prof["steps"] = prof.get("steps", 0) + 1
        return out

    def set_prefill_rows(self, rows: int) -> None:
        abi.check(self.L.smk_llama_set_prefill_rows(self.h, rows), "smk_llama_set_prefill_rows")

    def generate(self, prompt: list[int], n_new: int) -> tuple[np.ndarray, float, float]:
        p = np.asarray(prompt, np.int32)
        out = np.empty(n_new, np.int32)
        sec = np.zeros(2, np.float64)
        abi.check(self.L.smk_llama_generate(self.h, p.ctypes.data, len(p), n_new, out.ctypes.data, sec.ctypes.data),
                  "smk_llama_generate")
        return out, float(sec[0]), float(sec[1])

    def close(self) -> None:
        if self.h:
            abi.check(self.L.smk_llama_destroy(self.h), "smk_llama_destroy")
            self.h = None


def config_from_gguf(g: ggufmod.GGUF) -> Config:
    """A Config from the GGUF's llama.* metadata (for files without a config.json)."""
    md = g.metadata
    if md.get("general.architecture") != "llama":
        raise ValueError(f"{g.path}: architecture {md.get('general.architecture')!r}, expected llama")
    heads = int(md["llama.attention.head_count"])
    hidden = int(md["llama.embedding_length"])
    rs = md.get("smk.rope_scaling")
    return Config(hidden_size=hidden, intermediate_size=int(md["llama.feed_forward_length"]),
                  num_hidden_layers=int(md["llama.block_count"]), num_attention_heads=heads,
                  num_key_value_heads=int(md.get("llama.attention.head_count_kv", heads)),
                  head_dim=int(md.get("llama.rope.dimension_count", hidden // heads)),
                  vocab_size=int(md.get("llama.vocab_size", g.tensors["token_embd.weight"].shape[0])),
                  # GGUF stores epsilon as float32: take the shortest decimal that rounds to it
                  # (1e-05, not 9.9999997e-06), which is what config.json holds.
                  rms_norm_eps=float(str(np.float32(md.get("llama.attention.layer_norm_rms_epsilon", 1e-5)))),
                  rope_theta=float(md.get("llama.rope.freq_base", 10000.0)),
                  rope_scaling=json.loads(rs) if isinstance(rs, str) else None,
                  tie_word_embeddings="output.weight" not in g.tensors)


# GGUF metadata keys that must agree with the configuration, and the Config field each mirrors.
_METADATA_FIELDS = (("llama.block_count", "num_hidden_layers"), ("llama.embedding_length", "hidden_size"),
                    ("llama.feed_forward_length", "intermediate_size"),
                    ("llama.attention.head_count", "num_attention_heads"),
                    ("llama.attention.head_count_kv", "num_key_value_heads"))


def _check_metadata(g: ggufmod.GGUF, cfg: Config, path: str) -> None:
    """The file must be a Llama GGUF whose shape metadata (where present) matches `cfg`; every
    disagreement is reported at once (the example's loader checks the same keys, llama.py:302-316)."""
    md = g.metadata
    arch = md.get("general.architecture")
    problems = [] if arch == "llama" else [f"general.architecture is {arch!r}, not 'llama'"]
    for key, field_name in _METADATA_FIELDS:
        expected = getattr(cfg, field_name)
        if key in md and int(md[key]) != expected:
            problems.append(f"{key} is {md[key]} where the configuration has {field_name} = {expected}")
    if problems:
        raise ValueError(f"{path} does not match the model configuration: " + "; ".join(problems))


# Weight-type names of the example's command line and the file-name suffix of each GGUF.
_GGUF_SUFFIX = {"fp32": "-F32.gguf", "q8_0": "-Q8_0.gguf", "q4_0": "-Q4_0.gguf"}


def find_gguf(model_dir: str, weights: str) -> str:
    """The GGUF of weight type `weights` in <model_dir>/gguf: the first, in name order, whose name
    ends with -F32 / -Q8_0 / -Q4_0 .gguf (the example's layout, llama.py:508-517)."""
    folder = os.path.join(model_dir, "gguf")
    suffix = _GGUF_SUFFIX[weights]
    names = sorted(n for n in (os.listdir(folder) if os.path.isdir(folder) else []) if n.endswith(suffix))
    if not names:
        raise FileNotFoundError(f"{folder} holds no file ending in {suffix} (weights={weights!r})")
    return os.path.join(folder, names[0])


# ─── synthetic models ────────────────────────────────────────────────────────

def synthetic_tensor_order(cfg: Config) -> list[tuple[str, tuple[int, ...]]]:
    """Names and shapes of the random matrices, in the order their values are drawn."""
    c = cfg
    d, f, hd = c.hidden_size, c.intermediate_size, c.head_dim
    order = [("token_embd.weight", (c.vocab_size, d))]
    if not c.tie_word_embeddings:
        order.append(("output.weight", (c.vocab_size, d)))
    for i in range(c.num_hidden_layers):
        order += [(f"blk.{i}.attn_q.weight", (c.num_attention_heads * hd, d)),
                  (f"blk.{i}.attn_k.weight", (c.num_key_value_heads * hd, d)),
                  (f"blk.{i}.attn_v.weight", (c.num_key_value_heads * hd, d)),
                  (f"blk.{i}.attn_output.weight", (d, c.num_attention_heads * hd)),
                  (f"blk.{i}.ffn_gate.weight", (f, d)), (f"blk.{i}.ffn_up.weight", (f, d)),
                  (f"blk.{i}.ffn_down.weight", (d, f))]
    return order


def write_synthetic_model(model_dir: str, config: dict, seed: int, n_prompt: int = 32, quantize=None,
                          weight_type: int = ggufmod.Q4_0, name: str = "synthetic") -> tuple[str, list[int]]:
    """A random-init Llama as GGUF + config.json in model_dir.  rng = default_rng(seed): first the
    n_prompt prompt ids (uniform in [0, vocab)), then every matrix N(0, 0.02) as float32 in
    synthetic_tensor_order, each quantized by `quantize` (default: this module's device quantizer,
    bit-exact with ggml's) to `weight_type`; norm weights are 1.0.  Returns (gguf path, prompt)."""
    cfg = Config.from_dict(config)
    rng = np.random.default_rng(seed)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab_size, n_prompt)]
    if quantize is None:
        quantize = sk.quantize_q4_0 if weight_type == ggufmod.Q4_0 else sk.quantize_q8_0

    def matrix(shape):
        def make():
            w = rng.standard_normal(shape, dtype=np.float32)
            w *= np.float32(0.02)
            return w if weight_type == ggufmod.F32 else quantize(w)
        return make

    ones = np.ones(cfg.hidden_size, np.float32)
    tensors = []
    for tname, shape in synthetic_tensor_order(cfg):
        tensors.append((tname, weight_type, shape, matrix(shape)))
        if tname.endswith("attn_q.weight"):
            i = tname.split(".")[1]
            tensors.append((f"blk.{i}.attn_norm.weight", ggufmod.F32, (cfg.hidden_size,), ones))
        if tname.endswith("ffn_gate.weight"):
            i = tname.split(".")[1]
            tensors.append((f"blk.{i}.ffn_norm.weight", ggufmod.F32, (cfg.hidden_size,), ones))
    tensors.append(("output_norm.weight", ggufmod.F32, (cfg.hidden_size,), ones))
    md = {
        "general.architecture": "llama", "general.name": name,
        "general.file_type": ("u32", {ggufmod.F32: 0, ggufmod.Q4_0: 2, ggufmod.Q8_0: 7}[weight_type]),
        "llama.block_count": ("u32", cfg.num_hidden_layers), "llama.context_length": ("u32", 131072),
        "llama.embedding_length": ("u32", cfg.hidden_size), "llama.feed_forward_length": ("u32", cfg.intermediate_size),
        "llama.attention.head_count": ("u32", cfg.num_attention_heads),
        "llama.attention.head_count_kv": ("u32", cfg.num_key_value_heads),
        "llama.rope.freq_base": float(cfg.rope_theta), "llama.rope.dimension_count": ("u32", cfg.head_dim),
        "llama.attention.layer_norm_rms_epsilon": float(cfg.rms_norm_eps),
        "llama.vocab_size": ("u32", cfg.vocab_size),
        "smk.rope_scaling": json.dumps(cfg.rope_scaling),
        "smk.synthetic_seed": ("u64", seed),
    }
    os.makedirs(os.path.join(model_dir, "gguf"), exist_ok=True)
    suffix = {ggufmod.F32: "F32", ggufmod.Q4_0: "Q4_0", ggufmod.Q8_0: "Q8_0"}[weight_type]
    path = os.path.join(model_dir, "gguf", f"{name}-{suffix}.gguf")
    ggufmod.write(path, md, tensors)
    ggufmod.write_config(model_dir, config)
    return path, prompt
