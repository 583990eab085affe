"""Writes tests/golden/llama_3_2_1b_q4_0_seed5.json: the greedy tokens of the reference's CPU
decode loop on the synthetic Llama-3.2-1B, 32-token prompt, 128 new tokens.

The model comes from oracle/llama_ref.synthetic_model (seed 5: prompt ids, then every matrix
N(0, 0.02) quantized to Q4_0 by the oracle's quantizer, norm weights 1.0).  The tokens are
decoded on the CPU with the reference's own kernel table (oracle/_ref, built from its sources;
the AVX-512 table where the CPU has it) and with the oracle's C restatement of that table's
arithmetic order ("simd"); the two must agree token for token (their logits are bit-identical).
The scalar table ("port") is decoded too and recorded: its different summation order flips
int8 activation quants (x is re-quantized before every GEMV) and its tokens part from the SIMD
tables' after a few steps, which is why the GPU path follows the SIMD order exactly.  Run from the repository root:

    python tests/golden/make_llama_tokens.py
"""

import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import llama_ref as lr  # noqa: E402
from oracle import oracle as o  # noqa: E402

CONFIG = {
    "model_type": "llama", "hidden_size": 2048, "intermediate_size": 8192, "num_hidden_layers": 16,
    "num_attention_heads": 32, "num_key_value_heads": 8, "head_dim": 64, "vocab_size": 128256,
    "rms_norm_eps": 1e-5, "rope_theta": 500000.0, "tie_word_embeddings": True, "hidden_act": "silu",
    "rope_scaling": {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                     "original_max_position_embeddings": 8192},
}
SEED, N_PROMPT, N_NEW = 5, 32, 128
OUT = os.path.join(ROOT, "tests", "golden", "llama_3_2_1b_q4_0_seed5.json")


def main() -> None:
    c = lr.Cfg.from_config(CONFIG)
    t = time.time()
    prompt, W = lr.synthetic_model(c, SEED, N_PROMPT)
    print(f"model generated in {time.time() - t:.1f} s", flush=True)
    runs = {}
    for kind in ("reference", "simd", "port"):
        if kind == "reference" and o.ref() is None:
            continue
        if kind == "reference":
            o.ref().ref_set_num_threads(len(os.sched_getaffinity(0)))
        t = time.time()
        ids, margins, _ = lr.Decoder(c, W, lr.Q4_0, kind).generate(prompt, N_NEW)
        runs[kind] = {"tokens": ids, "top2_margin": [round(m, 6) for m in margins]}
        print(f"{kind}: {time.time() - t:.1f} s, min margin {min(margins):.4g}, first {ids[:8]}", flush=True)
    kinds = [k for k in runs if k != "port"]
    for k in kinds[1:]:
        assert runs[k]["tokens"] == runs[kinds[0]]["tokens"], f"{k} tokens differ from {kinds[0]}"
    if "port" in runs:
        same = [a == b for a, b in zip(runs["port"]["tokens"], runs[kinds[0]]["tokens"])]
        runs["port"]["first_difference"] = same.index(False) if False in same else None
    doc = {"config": CONFIG, "seed": SEED, "weight_type": "Q4_0", "prompt": prompt, "n_new": N_NEW,
           "stop_at_eos": False, "recipe": "oracle/llama_ref.synthetic_model",
           "reference_isa": o.ref_best_isa() if "reference" in runs else None,
           "tokens": runs[kinds[0]]["tokens"], "runs": runs}
    with open(OUT, "w") as f:
        json.dump(doc, f)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
