"""GPU parity of the Llama decode loop against the reference's CPU loop.

* Tiny models: the device engine's greedy tokens equal the reference loop's
  (oracle/llama_ref.py with the reference's own kernels when oracle/_ref is built, else the
  oracle's restatement of their order).  With Q4_0 matrices every logit is bit-identical at
  every step (GEMV, attention, softmax and SiLU follow the reference's SIMD order; RMSNorm and
  RoPE its numpy code); with Q8_0 / F32 matrices the logits stay within 2e-4.  The
  module-call loop (device_loop=False) gives the same tokens and logits within 2e-4.
* Llama-3.2-1B shape, seed 5, Q4_0: 32-token prompt and 128 greedy tokens equal the committed
  tokens of the reference's CPU loop (tests/golden/make_llama_tokens.py).
"""

import json
import os

import numpy as np
import pytest

from oracle import llama_ref as lr
from oracle import oracle as o
from simd_ml_kernels import gguf, llama

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
TINY = {"model_type": "llama", "hidden_size": 256, "intermediate_size": 512, "num_hidden_layers": 2,
        "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 64, "vocab_size": 1000,
        "rms_norm_eps": 1e-5, "rope_theta": 500000.0, "tie_word_embeddings": True,
        "rope_scaling": {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                         "original_max_position_embeddings": 8192}}
WTYPES = {"q4_0": (gguf.Q4_0, lr.Q4_0), "q8_0": (gguf.Q8_0, lr.Q8_0), "f32": (gguf.F32, lr.F32)}


def _oracle_kind():
    return "reference" if o.ref() is not None and o.ref_best_isa() in ("avx2", "avx512") else "simd"


def _tiny(tmp_path, wname, seed=21, n_prompt=8):
    gtype, ltype = WTYPES[wname]
    path, prompt = llama.write_synthetic_model(str(tmp_path), TINY, seed=seed, n_prompt=n_prompt, weight_type=gtype)
    c = lr.Cfg.from_config(TINY)
    oprompt, W = lr.synthetic_model(c, seed, n_prompt, ltype)
    assert prompt == oprompt
    return path, prompt, lr.Decoder(c, W, ltype, _oracle_kind())


@pytest.mark.parametrize("wname", ["q4_0", "q8_0", "f32"])
def test_tiny_engine_matches_reference_loop(tmp_path, wname):
    path, prompt, dec = _tiny(tmp_path, wname)
    ids_ref, margins, _ = dec.generate(prompt, 16)
    m = llama.Llama(str(tmp_path), gguf=path)
    try:
        ids = list(m.generate(prompt, 16, stop_at_eos=False))
        assert ids == ids_ref, (ids, ids_ref, margins)
        # Teacher-forced: logits of every position against the reference loop.
        seq = prompt + ids_ref[:-1]
        m.reset(len(seq))
        dec.reset(len(seq))
        for i, t in enumerate(seq):
            lg = m.step(t)
            lo = dec.step(t)
            if wname == "q4_0":
                np.testing.assert_array_equal(lg.view(np.uint32), lo.view(np.uint32), err_msg=f"position {i}")
            else:
                assert np.abs(lg - lo).max() <= 2e-4, np.abs(lg - lo).max()
            assert int(np.argmax(lg)) == int(np.argmax(lo))
    finally:
        m.close()


def test_tiny_long_context_several_attention_rounds(tmp_path):
    """A cache of 600 positions is read in rounds of 256 (the K / V tiles); logits stay
    bit-identical with the reference loop past the first round."""
    path, prompt, dec = _tiny(tmp_path, "q4_0", seed=26)
    rng = np.random.default_rng(26)
    seq = prompt + [int(t) for t in rng.integers(0, TINY["vocab_size"], 292)]
    m = llama.Llama(str(tmp_path), gguf=path)
    try:
        m.reset(600)
        dec.reset(600)
        for i, t in enumerate(seq):
            lg = m.step(t)
            lo = dec.step(t)
            if i >= 240 or i % 37 == 0:
                np.testing.assert_array_equal(lg.view(np.uint32), lo.view(np.uint32), err_msg=f"position {i}")
    finally:
        m.close()


@pytest.mark.parametrize("head_dim,heads,kv_heads", [(128, 4, 2), (256, 2, 1)])
def test_wide_heads_several_attention_rounds(tmp_path, head_dim, heads, kv_heads):
    """head_dim 128 (Llama-3-8B) and 256 (the engine's limit): the attention kernel's K / V tiles
    then hold fewer positions than at head_dim 64, so a 400-position cache takes several rounds.
    Logits bit-identical with the reference loop at positions across every round."""
    cfg = dict(TINY, hidden_size=heads * head_dim, intermediate_size=2 * heads * head_dim,
               num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=head_dim)
    path, prompt = llama.write_synthetic_model(str(tmp_path), cfg, seed=31 + head_dim, n_prompt=8,
                                               weight_type=gguf.Q4_0)
    c = lr.Cfg.from_config(cfg)
    oprompt, W = lr.synthetic_model(c, 31 + head_dim, 8, lr.Q4_0)
    assert prompt == oprompt
    dec = lr.Decoder(c, W, lr.Q4_0, _oracle_kind())
    rng = np.random.default_rng(head_dim)
    seq = prompt + [int(t) for t in rng.integers(0, cfg["vocab_size"], 392)]
    m = llama.Llama(str(tmp_path), gguf=path)
    try:
        m.reset(len(seq))
        dec.reset(len(seq))
        for i, t in enumerate(seq):
            lg = m.step(t)
            lo = dec.step(t)
            if i % 23 == 0 or i >= len(seq) - 3:
                np.testing.assert_array_equal(lg.view(np.uint32), lo.view(np.uint32), err_msg=f"position {i}")
    finally:
        m.close()


MID = dict(TINY, hidden_size=2048, intermediate_size=8192, num_attention_heads=32, num_key_value_heads=8,
           head_dim=64)


@pytest.mark.parametrize("tiles", [0, 2])
def test_mid_model_logits_equal_reference_loop(tmp_path, tiles):
    """Llama-3.2-1B layer widths (K = 2048 and 8192, the shapes of the fused GEMV launches) with
    two layers: logits bit-identical with the reference loop at every position, through the fused
    RMSNorm prologues and the SiLU and residual epilogues.  tiles = 2 forces the K-chunk tiled
    kernel wherever it applies (smk_set_q4_tiles): the lm_head and q|k|v then take its fused-norm
    prologue, o and down its plain form."""
    from simd_ml_kernels import abi
    path, prompt = llama.write_synthetic_model(str(tmp_path), MID, seed=27, n_prompt=6, weight_type=gguf.Q4_0)
    c = lr.Cfg.from_config(MID)
    oprompt, W = lr.synthetic_model(c, 27, 6, lr.Q4_0)
    assert prompt == oprompt
    dec = lr.Decoder(c, W, lr.Q4_0, _oracle_kind())
    seq = prompt + [11, 222, 333]
    abi.call("smk_set_q4_tiles", tiles)
    m = llama.Llama(str(tmp_path), gguf=path)
    try:
        m.reset(len(seq))
        dec.reset(len(seq))
        for i, t in enumerate(seq):
            np.testing.assert_array_equal(m.step(t).view(np.uint32), dec.step(t).view(np.uint32),
                                          err_msg=f"position {i}, tiles {tiles}")
    finally:
        m.close()
        abi.call("smk_set_q4_tiles", 0)


@pytest.mark.parametrize("wname,model,rows", [("q4_0", "tiny", 64), ("q4_0", "tiny", 3), ("q8_0", "tiny", 5),
                                              ("q4_0", "mid", 4), ("q4_0", "mid", 64)])
def test_chunked_prefill_equals_token_by_token(tmp_path, wname, model, rows):
    """The prompt in chunks of rows (matrix-core products over the rows, one attention launch per
    chunk) leaves the same KV cache and first token as one decode step per prompt token: the
    generated tokens match, and so does every bit of a further step's logits, which read the
    whole cache."""
    cfg = TINY if model == "tiny" else MID
    gtype, _ = WTYPES[wname]
    path, prompt = llama.write_synthetic_model(str(tmp_path), cfg, seed=31, n_prompt=11, weight_type=gtype)
    m = llama.Llama(str(tmp_path), gguf=path)
    try:
        out = {}
        for r in (0, rows):
            m.set_prefill_rows(r)
            ids = list(m.generate(prompt, 6, stop_at_eos=False))
            out[r] = (ids, m.step(ids[-1]))
        assert out[0][0] == out[rows][0]
        np.testing.assert_array_equal(out[0][1].view(np.uint32), out[rows][1].view(np.uint32))
    finally:
        m.close()


def test_tiny_module_loop_matches_engine(tmp_path):
    path, prompt, _ = _tiny(tmp_path, "q4_0", seed=22)
    eng = llama.Llama(str(tmp_path), gguf=path)
    host = llama.Llama(str(tmp_path), gguf=path, device_loop=False)
    try:
        seq = prompt + [5, 17, 999, 0]
        eng.reset(len(seq))
        host.reset(len(seq))
        for t in seq:
            a, b = eng.step(t), host.step(t)
            assert np.abs(a - b).max() <= 2e-4
        assert list(eng.generate(prompt, 10, stop_at_eos=False)) == list(host.generate(prompt, 10, stop_at_eos=False))
        # logits=False skips the lm_head and still advances the position.
        eng.reset(4)
        assert eng.step(prompt[0], logits=False) is None and eng.pos == 1
    finally:
        eng.close()
        host.close()


def test_tiny_generate_stops_at_eos_and_reports_stats(tmp_path):
    path, prompt, dec = _tiny(tmp_path, "q4_0", seed=23)
    ids_ref, _, _ = dec.generate(prompt, 12)
    m = llama.Llama(str(tmp_path), gguf=path)
    try:
        m.cfg.eos_token_ids = (ids_ref[3],)
        stats = {}
        ids = list(m.generate(prompt, 12, stats=stats))
        assert ids == ids_ref[:ids_ref.index(ids_ref[3]) + 1]
        assert stats["prefill_tokens"] == len(prompt) and stats["decode_steps"] == 11 and stats["decode_s"] > 0
    finally:
        m.close()


def test_engine_rejects_bad_calls(tmp_path):
    path, prompt, _ = _tiny(tmp_path, "q4_0", seed=24)
    m = llama.Llama(str(tmp_path), gguf=path)
    try:
        with pytest.raises(RuntimeError):
            m.step(0)  # no reset yet
        m.reset(2)
        with pytest.raises(RuntimeError):
            m._engine.step(1000, True)  # token out of range (vocab 1000)
        m.step(1)
        m.step(2)
        with pytest.raises(ValueError):
            m.step(3)  # cache full
    finally:
        m.close()


def test_llama_3_2_1b_greedy_tokens_equal_reference(tmp_path):
    """32-token prompt, 128 greedy tokens, token-identical with the
    reference's CPU loop on the same seeded model."""
    with open(os.path.join(HERE, "golden", "llama_3_2_1b_q4_0_seed5.json")) as f:
        gold = json.load(f)
    print(f"writing the synthetic Llama-3.2-1B (seed {gold['seed']})", flush=True)
    path, prompt = llama.write_synthetic_model(str(tmp_path), gold["config"], seed=gold["seed"],
                                               n_prompt=len(gold["prompt"]))
    assert prompt == gold["prompt"]
    m = llama.Llama(str(tmp_path), gguf=path)
    try:
        stats = {}
        ids = list(m.generate(prompt, gold["n_new"], stats=stats, stop_at_eos=False))
        print(f"decode {stats['decode_steps'] / stats['decode_s']:.1f} tok/s", flush=True)
        assert ids == gold["tokens"]
    finally:
        m.close()
