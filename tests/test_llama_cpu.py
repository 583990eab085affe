"""CPU checks of the decode-loop host side: the GGUF reader/writer, the synthetic-model recipe
(product writer against the oracle's independent generator, byte for byte), the RoPE tables,
and the oracle's restated decode loop against the reference's own kernels and float64."""

import json
import os

import numpy as np
import pytest

from oracle import llama_ref as lr
from oracle import oracle as o
from simd_ml_kernels import gguf, llama

TINY = {"model_type": "llama", "hidden_size": 256, "intermediate_size": 512, "num_hidden_layers": 2,
        "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 64, "vocab_size": 1000,
        "rms_norm_eps": 1e-5, "rope_theta": 500000.0, "tie_word_embeddings": True,
        "rope_scaling": {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                         "original_max_position_embeddings": 8192}}


class TestGGUF:
    def test_round_trip_every_type(self, tmp_path):
        rng = np.random.default_rng(0)
        w = rng.standard_normal((6, 64)).astype(np.float32)
        q4, q8 = o.quantize_q4_0(w), o.quantize_q8_0(w)
        f16 = w.astype(np.float16)
        bf16 = o.to_bf16_rne(w)
        md = {"general.architecture": "llama", "x.i32": -5, "x.f32": 1.5, "x.u32": ("u32", 7),
              "x.u64": ("u64", 2 ** 40), "x.f64": ("f64", 0.1), "x.str": "héllo", "x.bool": True}
        path = str(tmp_path / "t.gguf")
        gguf.write(path, md, [("a", gguf.F32, w.shape, w), ("b", gguf.Q4_0, w.shape, q4),
                              ("c", gguf.Q8_0, w.shape, lambda: q8), ("d", gguf.F16, w.shape, f16),
                              ("e", gguf.BF16, w.shape, bf16), ("v", gguf.F32, (64,), w[0])])
        g = gguf.GGUF(path)
        assert g.version == 3 and g.metadata["x.i32"] == -5 and g.metadata["x.str"] == "héllo"
        assert g.metadata["x.u64"] == 2 ** 40 and g.metadata["x.bool"] is True and g.metadata["x.f64"] == 0.1
        np.testing.assert_array_equal(g.tensors["a"].data, w)
        np.testing.assert_array_equal(g.tensors["b"].data, q4)
        np.testing.assert_array_equal(g.tensors["c"].data, q8)
        np.testing.assert_array_equal(g.tensors["d"].data, f16)
        np.testing.assert_array_equal(g.tensors["e"].data, bf16)
        assert g.tensors["v"].shape == (64,) and g.tensors["b"].shape == (6, 64)
        for name in "abcde":
            assert not g.tensors[name].data.flags.writeable  # read-only: device-resident after first use
            assert g.tensors[name].data.ctypes.data % 32 == 0

    def test_dequantize_rows(self, tmp_path):
        rng = np.random.default_rng(1)
        w = rng.standard_normal((5, 96)).astype(np.float32)
        for t, data in ((gguf.Q4_0, o.quantize_q4_0(w)), (gguf.Q8_0, o.quantize_q8_0(w))):
            tens = gguf.Tensor("t", t, (5, 96), data)
            ref = lr.dequant(lr.Q4_0 if t == gguf.Q4_0 else lr.Q8_0, data, 5, 96)
            np.testing.assert_array_equal(gguf.dequantize_rows(tens, [3, 0]), ref[[3, 0]])
            assert np.abs(gguf.dequantize_rows(tens, 2)[0] - w[2]).max() < 0.3

    def test_rejects_non_gguf_and_bad_type(self, tmp_path):
        p = tmp_path / "x.gguf"
        p.write_bytes(b"NOPE" + b"\0" * 64)
        with pytest.raises(ValueError, match="magic"):
            gguf.GGUF(str(p))

    def test_malformed_files(self, tmp_path):
        """Version, value kind, truncation, unknown tensor type and a tensor past the end are all
        refused with ValueError; string and numeric arrays are read."""
        import struct

        def header(n_tensors, pairs, version=3):
            return b"GGUF" + struct.pack("<IQQ", version, n_tensors, len(pairs)) + b"".join(pairs)

        def key(k):
            return struct.pack("<Q", len(k)) + k.encode()

        cases = {
            "v1.gguf": (header(0, [], version=1), "version 1"),
            "kind.gguf": (header(0, [key("a") + struct.pack("<I", 13) + b"\0" * 8]), "kind 13"),
            "short.gguf": (header(0, [key("a") + struct.pack("<IQ", 8, 100) + b"xy"]), "truncated"),
            "type.gguf": (header(1, []) + key("t") + struct.pack("<IQIQ", 1, 32, 6, 0) + b"\0" * 64, "ggml type 6"),
            "past.gguf": (header(1, []) + key("t") + struct.pack("<IQIQ", 1, 4096, 0, 0) + b"\0" * 64, "needs bytes"),
        }
        for name, (blob, msg) in cases.items():
            p = tmp_path / name
            p.write_bytes(blob)
            with pytest.raises(ValueError, match=msg):
                gguf.GGUF(str(p))
        names = key("names") + struct.pack("<IIQ", 9, 8, 2) + struct.pack("<Q", 2) + b"ab" + struct.pack("<Q", 1) + b"c"
        ids = key("ids") + struct.pack("<IIQ", 9, 5, 3) + struct.pack("<3i", 7, -1, 9)
        p = tmp_path / "arr.gguf"
        p.write_bytes(header(0, [names, ids]))
        g = gguf.GGUF(str(p))
        assert g.metadata["names"] == ["ab", "c"] and list(g.metadata["ids"]) == [7, -1, 9]


class TestSyntheticRecipe:
    def test_product_writer_matches_oracle_generator(self, tmp_path):
        """Same seed -> same prompt and byte-identical Q4_0 tensors (the writer takes the oracle's
        quantizer here; on the GPU it uses the library's, which is byte-exact with it)."""
        path, prompt = llama.write_synthetic_model(str(tmp_path), TINY, seed=3, n_prompt=8,
                                                   quantize=o.quantize_q4_0)
        c = lr.Cfg.from_config(TINY)
        oprompt, W = lr.synthetic_model(c, 3, 8)
        assert prompt == oprompt
        g = gguf.GGUF(path)
        np.testing.assert_array_equal(g.tensors["token_embd.weight"].data, W["token_embd"])
        for i in range(c.n_layers):
            for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"):
                np.testing.assert_array_equal(g.tensors[f"blk.{i}.{n}.weight"].data, W[f"{i}.{n}"])
            np.testing.assert_array_equal(g.tensors[f"blk.{i}.attn_norm.weight"].data, np.ones(256, np.float32))
        assert json.load(open(os.path.join(str(tmp_path), "config.json")))["hidden_size"] == 256
        cfg = llama.config_from_gguf(g)
        assert cfg == llama.Config.from_dict(TINY)

    def test_rope_tables_equal_oracle(self):
        cfg = llama.Config.from_dict(TINY)
        inv = llama.rope_inv_freq(cfg)
        np.testing.assert_array_equal(inv, o.rope_inv_freq(64, 500000.0, TINY["rope_scaling"]))
        cos, sin = llama.rope_tables(inv, 40)
        for p in (0, 1, 39):
            c, s = o.rope_cos_sin(inv, p)
            np.testing.assert_array_equal(cos[p], c)
            np.testing.assert_array_equal(sin[p], s)

    def test_config_checks(self):
        with pytest.raises(ValueError):
            llama.Config.from_dict({**TINY, "model_type": "mistral"})
        with pytest.raises(ValueError):
            llama.Config.from_dict({**TINY, "attention_bias": True})


class TestOracleDecodeLoop:
    """The restated loop (oracle/llama_ref.py) against the reference's own kernels and float64."""

    @pytest.mark.parametrize("wtype", [lr.Q4_0, lr.Q8_0])
    def test_reference_port_and_f64_agree(self, wtype, ref_lib):
        c = lr.Cfg.from_config(TINY)
        prompt, W = lr.synthetic_model(c, 11, 8, wtype)
        runs = {k: lr.Decoder(c, W, wtype, k).generate(prompt, 12) for k in ("reference", "port", "f64")}
        ids_ref, m_ref, lg_ref = runs["reference"]
        assert runs["port"][0] == ids_ref
        assert min(m_ref) > 1e-3
        # The port is the reference's scalar semantics; logits within a few fp32 roundings.
        np.testing.assert_allclose(runs["port"][2], lg_ref, atol=2e-4)
        # float64 without activation quantization: same greedy ids where the margin is wide.
        for a, b, m in zip(runs["f64"][0], ids_ref, m_ref):
            if m > 0.05:
                assert a == b

    def test_planted_rope_mistake_changes_logits(self):
        c = lr.Cfg.from_config(TINY)
        prompt, W = lr.synthetic_model(c, 12, 4)
        good = lr.Decoder(c, W, lr.Q4_0, "port")
        bad = lr.Decoder(c, W, lr.Q4_0, "port")
        bad.inv_freq = bad.inv_freq[::-1].copy()  # frequencies reversed
        _, _, a = good.generate(prompt, 3)
        _, _, b = bad.generate(prompt, 3)
        assert np.abs(a - b).max() > 1e-3


def test_device_loop_fails_loudly_without_gpu(tmp_path):
    """No CPU fallback: the engine refuses to start without a gfx950 device."""
    from simd_ml_kernels import abi
    rc_dev = abi.lib().smk_device_info(None, 0, None, 0, None, None)
    if rc_dev == 0:
        pytest.skip("a GPU is present")
    path, _ = llama.write_synthetic_model(str(tmp_path), TINY, seed=1, n_prompt=4, quantize=o.quantize_q4_0)
    with pytest.raises(RuntimeError):
        llama.Llama(str(tmp_path), gguf=path)
