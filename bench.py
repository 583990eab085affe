#!/usr/bin/env python3
"""Benchmark of the MI355X decode-GEMV path (one GPU).

Headline (BASELINE.json metric "Q4_0 GEMV weight GB/s & % of HBM peak"): the Q4_0
decode GEMV y = x @ W.T at the Llama-3.2-1B FFN up/gate shape N=8192, K=2048
x ~ N(0,1), W ~ N(0,0.02) quantized to GGUF Q4_0 by this
library's bit-exact quantizer, seed 0, summed in the reference's SIMD order (y bit-exact
with its AVX2 / AVX-512 tables).  A step is one GEMV launch on the next of
ceil(512 MiB / 9.4 MB) + 1 distinct device copies of W, so the 256 MB Infinity
Cache never holds the weights; inputs are resident in HBM before timing starts.
Steps are launched back to back on one stream and timed with HIP events recorded
on that same stream; the launch loop is captured in a HIP graph (mode "graph",
default) or issued from Python (mode "stream").

The JSON line also carries the other GEMV configurations (Q8_0 both orientations,
FP16/BF16 and Q4_0 at Llama-3-8B shapes, the Q4_0 lm_heads, the Llama-3.2-1B decode
shapes, batched rows M = 2, 4, 8, the headline shape in free summation order), the
measured HBM read roof, the roofline of the headline kernel, the decode of BASELINE
config 5 (128 greedy tokens of the synthetic Llama-3.2-1B through the device engine,
token-checked against the reference's CPU loop) and the CPU baseline: the REFERENCE's
own best SIMD path (oracle/_ref, built from its sources) on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "simd-ml-kernels_amd"))

import numpy as np  # noqa: E402

PEAK_HBM = 8.0e12  # MI355X published HBM3E bandwidth, bytes/s
ROTATE_BYTES = 512 * 2 ** 20
BB = {"q4_0": 18, "q8_0": 34}


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000, help="timed GEMV launches of the headline case")
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--mode", choices=["graph", "stream"], default="graph")
    p.add_argument("--cases", choices=["all", "headline", "decode", "batched", "decode-eager"], default="all",
                   help="decode: only the decode model; batched: only the config 4 Q4_0 products "
                        "(M = 1, 2, 4, 8, 32 at 14336x4096, both kernels); decode-eager: only the decode "
                        "model, its 159 positions stepped one kernel at a time with per-section events "
                        "(a profiler-friendly breakdown)")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


class Dev:
    """Device buffers, a stream, events and graphs, all through the library's C ABI (no other
    GPU framework is loaded, so the process runs the HIP runtime the library was built for)."""

    def __init__(self):
        from simd_ml_kernels import abi
        self.abi = abi
        self.L = abi.lib()
        self.stream = abi.Stream()  # default priority
        self.sp = self.stream.handle

    def put(self, a: np.ndarray):
        return self.abi.Buffer.of(a)

    def empty(self, nbytes: int):
        return self.abi.Buffer(max(nbytes, 16))

    def sync(self):
        self.abi.call("smk_synchronize")

    def quantize(self, fmt: str, w_dev, rows: int, K: int):
        out = self.empty(rows * (K // 32) * BB[fmt])
        bad = self.abi.Buffer.filled(4, 0)
        self.abi.call("smk_d_quantize", BB[fmt], rows, K, w_dev.ptr, out.ptr, bad.ptr, self.sp)
        self.sync()
        assert int(bad.numpy(np.int32)[0]) == 0
        return out

    def clone(self, buf):
        out = self.abi.Buffer(buf.nbytes)
        self.abi.call("smk_memcpy_d2d", out.ptr, buf.ptr, buf.nbytes)
        return out

    def timed(self, fn, reps: int) -> float:
        """Seconds for fn() (which enqueues on self.stream) run reps times, HIP events on the stream."""
        a, b = self.abi.Event(), self.abi.Event()
        a.record(self.stream)
        for _ in range(reps):
            fn()
        b.record(self.stream)
        return a.elapsed_ms(b) * 1e-3


def time_launches(dev: Dev, launch, n_copies: int, steps: int, warmup: int, mode: str) -> float:
    """Average seconds per launch over `steps` launches, HIP events on the launch stream."""
    for i in range(warmup):
        launch(i % n_copies)
    dev.stream.synchronize()
    if mode == "graph":
        per_graph = n_copies * max(1, 256 // n_copies) if n_copies < 256 else n_copies
        with dev.abi.Graph.capture(dev.stream) as cap:
            for i in range(per_graph):
                launch(i % n_copies)
        g = cap.graph
        reps = max(1, steps // per_graph)
        g.launch(dev.stream)
        dev.stream.synchronize()
        return dev.timed(lambda: g.launch(dev.stream), reps) / (reps * per_graph)
    it = iter(range(steps))
    return dev.timed(lambda: launch(next(it) % n_copies), steps) / steps


def quant_case(dev: Dev, fmt: str, N: int, K: int, seed: int, steps: int, warmup: int, mode: str, M: int = 1):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K), dtype=np.float32)
    w = rng.standard_normal((N, K), dtype=np.float32)
    w *= np.float32(0.02)
    wq = dev.quantize(fmt, dev.put(w), N, K)
    del w
    nbytes = N * (K // 32) * BB[fmt]
    copies = [wq] + [dev.clone(wq) for _ in range(math.ceil(ROTATE_BYTES / nbytes))]
    xd, yd = dev.put(x), dev.empty(4 * M * N)
    fn = dev.L.smk_d_gemm_q4_0 if fmt == "q4_0" else dev.L.smk_d_gemm_q8_0
    args = [(M, N, K, xd.ptr, K, c.ptr, yd.ptr, N, dev.sp) for c in copies]

    def launch(i):
        rc = fn(*args[i])
        if rc:
            dev.abi.check(rc, "gemm")

    sec = time_launches(dev, launch, len(copies), steps, warmup, mode)
    del copies
    return {"fmt": fmt, "M": M, "N": N, "K": K, "us": sec * 1e6, "weight_bytes": nbytes,
            "weight_GBps": nbytes / sec / 1e9, "pct_hbm_peak": 100 * nbytes / sec / PEAK_HBM,
            "GBps_weights_x_y": (nbytes + 4 * M * (K + N)) / sec / 1e9, "GFLOPs": 2 * M * N * K / sec / 1e9}


def batched_cases(dev: Dev, steps: int, warmup: int, mode: str) -> dict:
    """Q4_0 at N=14336, K=4096 for M = 2, 4, 8, 32 rows of x (M = 1 is the
    q4_0_14336x4096 case), each through the built-in choice (the int8 matrix-core kernel from
    M = 3 at this N) and through launches of 8 GEMV rows, the switch point's other side."""
    out = {}
    for M in (2, 4, 8, 32):
        out[f"q4_0_M{M}_14336x4096"] = quant_case(dev, "q4_0", 14336, 4096, 4, steps, warmup, mode, M=M)
        dev.abi.call("smk_set_q4_mfma_min_rows", 1 << 30)
        try:
            out[f"q4_0_M{M}_14336x4096_gemv_rows"] = quant_case(dev, "q4_0", 14336, 4096, 4, max(40, steps // 4),
                                                                10, mode, M=M)
        finally:
            dev.abi.call("smk_set_q4_mfma_min_rows", 0)
    return out


def lowp_case(dev: Dev, fmt: str, N: int, K: int, seed: int, steps: int, warmup: int, mode: str):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(K, dtype=np.float32)
    w = rng.standard_normal((N, K), dtype=np.float32)
    w *= np.float32(0.02)
    if fmt == "f16":
        xb, wb, elem = x.astype(np.float16).view(np.uint16), w.astype(np.float16).view(np.uint16), 1
    else:  # bf16 by truncation, as the reference bench (_cli.py:236-238)
        xb, wb, elem = (x.view(np.uint32) >> 16).astype(np.uint16), (w.view(np.uint32) >> 16).astype(np.uint16), 2
    del w
    wd = dev.put(wb)
    nbytes = wb.nbytes
    del wb
    copies = [wd] + [dev.clone(wd) for _ in range(math.ceil(ROTATE_BYTES / nbytes))]
    xd, yd = dev.put(xb), dev.empty(4 * N)
    args = [(elem, 1, N, K, 1.0, xd.ptr, K, c.ptr, K, 0.0, yd.ptr, N, dev.sp) for c in copies]
    fn = dev.L.smk_d_gemm_tb

    def launch(i):
        rc = fn(*args[i])
        if rc:
            dev.abi.check(rc, "gemm_tb")

    sec = time_launches(dev, launch, len(copies), steps, warmup, mode)
    del copies
    return {"fmt": fmt, "M": 1, "N": N, "K": K, "us": sec * 1e6, "weight_bytes": nbytes,
            "weight_GBps": nbytes / sec / 1e9, "pct_hbm_peak": 100 * nbytes / sec / PEAK_HBM,
            "GFLOPs": 2 * N * K / sec / 1e9}


def read_roof(dev: Dev, nbytes: int = 2 << 30, reps: int = 20, nontemporal: int = 0) -> float:
    """Bytes/s of the library's HBM read-stream kernel over a 2 GiB buffer."""
    src = dev.abi.Buffer.filled(nbytes, 1)
    sink = dev.empty(4 * 4096)
    run = lambda: dev.abi.call("smk_d_read_roof", src.ptr, nbytes, sink.ptr, nontemporal, dev.sp)
    for _ in range(3):
        run()
    dev.stream.synchronize()
    sec = dev.timed(run, reps)
    del src
    return nbytes * reps / sec


def copy_roof(dev: Dev, nbytes: int = 256 << 20, reps: int = 5) -> float:
    """Bytes/s (read + write) of the library's plain copy kernel over 256 MiB.  Under a PMC run its
    FETCH_SIZE and WRITE_SIZE per dispatch calibrate the counters: it moves exactly nbytes each way."""
    src = dev.abi.Buffer.filled(nbytes, 3)
    dst = dev.empty(nbytes)
    run = lambda: dev.abi.call("smk_d_copy", dst.ptr, src.ptr, nbytes, dev.sp)
    run()
    dev.stream.synchronize()
    sec = dev.timed(run, reps)
    del src, dst
    return 2 * nbytes * reps / sec


GOLDEN_TOKENS = os.path.join(ROOT, "tests", "golden", "llama_3_2_1b_q4_0_seed5.json")


def decode_case(runs: int = 3) -> dict:
    """the synthetic Llama-3.2-1B (seed 5, Q4_0, written as GGUF by the library's
    own writer and quantizer) through the device decode engine: 32-token prompt, 128 greedy tokens
    (stop_at_eos=False), `runs` times; tok/s = decode steps / decode time (HIP events around the
    127 graph-launched decode steps, as the reference's run_ours times its decode steps)."""
    import shutil
    import tempfile

    from simd_ml_kernels import llama

    with open(GOLDEN_TOKENS) as f:
        gold = json.load(f)
    tmp = tempfile.mkdtemp(prefix="smk_llama_", dir="/tmp")
    try:
        t = time.perf_counter()
        path, prompt = llama.write_synthetic_model(tmp, gold["config"], seed=gold["seed"],
                                                   n_prompt=len(gold["prompt"]))
        t_write = time.perf_counter() - t
        m = llama.Llama(tmp, gguf=path)
        try:
            list(m.generate(prompt[:8], 16, stop_at_eos=False))  # warm-up
            tps, pre = [], []
            ids = None
            for _ in range(runs):
                st = {}
                ids = list(m.generate(prompt, gold["n_new"], stats=st, stop_at_eos=False))
                tps.append(st["decode_steps"] / st["decode_s"])
                pre.append(st["prefill_s"] / st["prefill_tokens"])
            # The prompt one graph step per token (the reference loop's prefill), for comparison.
            m.set_prefill_rows(0)
            pre_tok = []
            ids_tok = None
            for _ in range(runs):
                st = {}
                ids_tok = list(m.generate(prompt, gold["n_new"], stats=st, stop_at_eos=False))
                pre_tok.append(st["prefill_s"] / st["prefill_tokens"])
            wb = m.weight_bytes()
        finally:
            m.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    tok_s = float(np.median(tps))
    return {"model": "Llama-3.2-1B architecture, random-init N(0,0.02), Q4_0 (tied token_embd as lm_head)",
            "prompt_tokens": len(prompt), "new_tokens": gold["n_new"], "decode_tok_s": round(tok_s, 1),
            "runs_tok_s": [round(v, 1) for v in tps], "ms_per_token": round(1e3 / tok_s, 4),
            "prefill_ms_per_token": round(1e3 * float(np.median(pre)), 4),
            "prefill": "one 32-row chunk: matrix-core Q4_0 products over the rows",
            "prefill_token_by_token_ms_per_token": round(1e3 * float(np.median(pre_tok)), 4),
            "tokens_equal_token_by_token_prefill": ids_tok == ids,
            "gemv_weight_bytes_per_token": int(wb),
            "gemv_weight_GBps": round(wb * tok_s / 1e9, 1), "pct_hbm_peak": round(100 * wb * tok_s / PEAK_HBM, 2),
            "tokens_match_reference_cpu_loop": ids == gold["tokens"], "model_write_s": round(t_write, 1)}


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemv_q4_0_8192x2048_hbm_traffic.md")


def profiled_traffic() -> int | None:
    """HBM bytes per launch of the headline kernel, from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by the copy/read-roof calibration)."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_baseline(N: int, K: int, budget_s: float) -> dict | None:
    """The reference's own gemv_q4_0 (widest table this CPU runs, OpenMP on every allowed core)
    on a bounded sample of the headline workload, weights rotated past the host caches."""
    from oracle import oracle as o  # the checker/baseline leg only
    cores = len(os.sched_getaffinity(0))
    R = o.ref()
    rng = np.random.default_rng(0)
    x = rng.standard_normal(K, dtype=np.float32)
    w = rng.standard_normal((N, K), dtype=np.float32)
    w *= np.float32(0.02)
    wq = o.quantize_q4_0(w)
    del w
    copies = [wq] + [wq.copy() for _ in range(math.ceil(ROTATE_BYTES / wq.nbytes))]
    y = np.zeros(N, np.float32)
    xp, yp = x.ctypes.data_as(o._f32p), y.ctypes.data_as(o._f32p)
    if R is not None:
        isa = o.ref_best_isa()
        R.ref_set_num_threads(cores)
        run = lambda c: R.ref_gemv_q4_0(o.ISA[isa], N, K, xp, c.ctypes.data_as(o._u8p), yp)
        kind, path, used = "reference", f"{isa} table, {R.ref_q8_0_path(o.ISA[isa]).decode()} inner loop", cores
    else:
        run = lambda c: o.lib().smko_gemv_q4_0(N, K, xp, c.ctypes.data_as(o._u8p), yp)
        kind, path, used = "port", "oracle C restatement (scalar)", 1
    for i in range(5):
        run(copies[i % len(copies)])
    times = []
    t_end = time.perf_counter() + budget_s
    i = 0
    while time.perf_counter() < t_end or len(times) < 30:
        t = time.perf_counter()
        run(copies[i % len(copies)])
        times.append(time.perf_counter() - t)
        i += 1
    med = float(np.median(times))
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next(line.split(":", 1)[1].strip() for line in f if line.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return {"value": wq.nbytes / med / 1e9, "unit": "GB/s", "cores": used, "kind": kind,
            "sample": f"{len(times)} gemv_q4_0 calls 8192x2048 (median {med * 1e6:.1f} us) over "
                      f"{len(copies)} rotated host copies ({len(copies) * wq.nbytes / 2 ** 20:.0f} MiB); {path}; {model}"}


def decode_eager() -> dict:
    """The decode model of decode_case, teacher-forced through its 159 positions (prompt + golden
    tokens) with eager, individually launched kernels and an event at each section start
    (smk_llama_step_profile): the per-section device time per token."""
    import shutil
    import tempfile

    from simd_ml_kernels import llama

    with open(GOLDEN_TOKENS) as f:
        gold = json.load(f)
    tmp = tempfile.mkdtemp(prefix="smk_llama_", dir="/tmp")
    try:
        path, prompt = llama.write_synthetic_model(tmp, gold["config"], seed=gold["seed"],
                                                   n_prompt=len(gold["prompt"]))
        m = llama.Llama(tmp, gguf=path)
        try:
            seq = prompt + gold["tokens"][:-1]
            m.profile = {}
            m.reset(len(seq))
            for t in seq:
                m.step(t)
            p = m.profile
        finally:
            m.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    n = p["steps"]
    return {"positions": n, "ms_per_token": round(1e3 * p["total"] / n, 4),
            "us_per_token": {k: round(1e6 * v / n, 1) for k, v in p["device"].items()}}


def main() -> int:
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}).", file=sys.stderr)
        return 2
    if args.cases == "decode-eager":
        print(json.dumps({"decode_eager": decode_eager()}))
        return 0
    if args.cases == "decode":
        print(json.dumps({"decode": decode_case()}))
        return 0
    dev = Dev()
    if args.cases == "batched":
        print(json.dumps({"batched": batched_cases(dev, max(200, args.steps // 4), 50, args.mode)}))
        return 0
    head = quant_case(dev, "q4_0", 8192, 2048, 0, args.steps, args.warmup, args.mode)
    cases = {}
    if args.cases == "all":
        st, wu = max(200, args.steps // 4), 50
        cases["q8_0_8192x2048"] = quant_case(dev, "q8_0", 8192, 2048, 1, st, wu, args.mode)
        cases["q8_0_2048x8192"] = quant_case(dev, "q8_0", 2048, 8192, 1, st, wu, args.mode)
        # The Llama-3-8B shapes of the north-star target (FFN up/gate, down, attention out).
        for fmt in ("q4_0", "q8_0"):
            for N, K in ((14336, 4096), (4096, 14336), (4096, 4096)):
                cases[f"{fmt}_{N}x{K}"] = quant_case(dev, fmt, N, K, 3, st, wu, args.mode)
        for fmt in ("f16", "bf16"):
            for N, K in ((14336, 4096), (4096, 14336), (4096, 4096)):
                cases[f"{fmt}_{N}x{K}"] = lowp_case(dev, fmt, N, K, 2, max(60, st // 8), 10, args.mode)
        cases["q4_0_lm_head_128256x4096"] = quant_case(dev, "q4_0", 128256, 4096, 3, 40, 4, args.mode)
        # The Llama-3.2-1B decode GEMVs (fused q|k|v, o, fused gate|up, down, lm_head) as plain calls.
        for N, K in ((3072, 2048), (2048, 2048), (16384, 2048), (2048, 8192)):
            cases[f"q4_0_{N}x{K}"] = quant_case(dev, "q4_0", N, K, 5, st, wu, args.mode)
        cases["q4_0_lm_head_128256x2048"] = quant_case(dev, "q4_0", 128256, 2048, 5, 60, 6, args.mode)
        # The headline shape with the free-order kernel (y within the reference's error bound, not
        # its bits): the cost of summing in the reference's SIMD order.
        dev.abi.call("smk_set_q4_order", 0)
        try:
            cases["q4_0_8192x2048_free_order"] = quant_case(dev, "q4_0", 8192, 2048, 0, st, wu, args.mode)
        finally:
            dev.abi.call("smk_set_q4_order", 1)
        cases.update(batched_cases(dev, st, wu, args.mode))
    roof = read_roof(dev, nontemporal=1)
    copy = copy_roof(dev)
    decode = decode_case() if args.cases == "all" else None
    sec = head["us"] * 1e-6
    achieved = head["weight_bytes"] / sec
    out = {
        "metric": "Q4_0 GEMV weight GB/s & % of HBM peak; decode tok/s at Llama-3.2-1B shape",
        "value": round(head["weight_GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["us"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xq4 (Q4_0 weights, Q8 activations, int32 block sums, fp32 accumulation)",
        "data": "synthetic: x~N(0,1), W~N(0,0.02) quantized to GGUF Q4_0, seed 0",
        "config": {"workload": "gemv_q4_0 N=8192 K=2048 (Llama-3.2-1B FFN up/gate, BASELINE config 1), "
                               f"{math.ceil(ROTATE_BYTES / head['weight_bytes']) + 1} rotated weight copies, "
                               f"launch mode {args.mode}"},
        "roofline": {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM, 4), "traffic": profiled_traffic(),
                     "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0)",
                     "algorithmic_bytes": head["weight_bytes"]},
        "pct_hbm_peak": round(100 * achieved / PEAK_HBM, 2),
        "hbm_read_roof_GBps": round(roof / 1e9, 1),
        "pct_read_roof": round(100 * achieved / roof, 2),
        "hbm_copy_GBps": round(copy / 1e9, 1),
        "GFLOPs": round(head["GFLOPs"], 1),
        "GBps_weights_x_y": round(head["GBps_weights_x_y"], 2),
        "cases": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                  for k, v in cases.items()},
    }
    if decode is not None:
        out["decode_tok_s"] = decode["decode_tok_s"]
        out["decode"] = decode
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(8192, 2048, args.cpu_seconds)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
