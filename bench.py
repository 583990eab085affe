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
    p.add_argument("--cases", choices=["all", "headline", "decode", "batched", "decode-eager", "shapes"],
                   default="all",
                   help="decode: only the decode model; batched: only the config 4 Q4_0 products "
                        "(M = 1, 2, 4, 8, 32 at 14336x4096, both kernels); decode-eager: only the decode "
                        "model, its 159 positions stepped one kernel at a time with per-section events "
                        "(a profiler-friendly breakdown); shapes: only the --shape GEMVs")
    p.add_argument("--shape", action="append", default=None, metavar="FMT:NxK",
                   help="with --cases shapes: a Q4_0 / Q8_0 / F16 / BF16 GEMV case, e.g. q4_0:14336x4096 "
                        "(repeatable; default the Llama-3-8B Q4_0 and Q8_0 shapes)")
    p.add_argument("--cpu-seconds", type=float, default=16.0,
                   help="budget of the CPU baseline's GEMV samples (the decode baseline adds a few seconds)")
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


FLUSH_BYTES = 1 << 30
RAMP_READS = 128  # x 1 GiB: about 20 ms at 7 TB/s


def time_launches(dev: Dev, launch, n_copies: int, steps: int, warmup: int, mode: str) -> float:
    """Average seconds per launch over exactly `steps` launches, HIP events on the launch stream.

    First about 20 ms of HBM reads (clock ramp), `warmup` launches, then (when `steps` launches
    cannot rotate through all the copies, i.e. fewer than ROTATE_BYTES of distinct weights) a 1 GiB
    read that evicts the caches, then the `steps` timed launches on copies the warm-up did not
    touch last, between two events.
    Graph mode captures the warm-up (with the eviction) and the timed launches as two graphs and
    records the events around the second one's launch; stream mode issues the launches from
    Python."""
    flush = dev.abi.Buffer.filled(FLUSH_BYTES, 5)
    sink = dev.empty(4 * 4096)

    def warm():
        # Clock ramp: ~20 ms of HBM reads before the warm-up launches (after an idle host gap
        # the first milliseconds of work run slower, which a few short launches would not absorb).
        for _ in range(RAMP_READS):
            dev.abi.call("smk_d_read_roof", flush.ptr, FLUSH_BYTES, sink.ptr, 0, dev.sp)
        for i in range(warmup):
            launch(i % n_copies)
        if steps < n_copies:  # the timed copies must not be in the caches
            dev.abi.call("smk_d_read_roof", flush.ptr, FLUSH_BYTES, sink.ptr, 0, dev.sp)

    def timed():
        for i in range(steps):
            launch((warmup + i) % n_copies)

    a, b = dev.abi.Event(), dev.abi.Event()
    launch(0)  # eager first call: a path's scratch (the batched product's) is sized outside any capture
    dev.stream.synchronize()
    if mode == "graph":
        with dev.abi.Graph.capture(dev.stream) as cap_w:
            warm()
        with dev.abi.Graph.capture(dev.stream) as cap_t:
            timed()
        gw, gt = cap_w.graph, cap_t.graph
        gw.launch(dev.stream)  # first replays: code objects and page tables warm
        gt.launch(dev.stream)
        dev.stream.synchronize()
        # The warm-up runs right before the timed launches, with no host wait between them: after
        # an idle gap the first launches run measurably slower (clocks ramp up again).
        gw.launch(dev.stream)
        a.record(dev.stream)
        gt.launch(dev.stream)
        b.record(dev.stream)
    else:
        warm()
        a.record(dev.stream)
        timed()
        b.record(dev.stream)
    dev.stream.synchronize()
    return a.elapsed_ms(b) * 1e-3 / steps


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


def decode_case(runs: int = 3, cpu: bool = False) -> dict:
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
        cpu_dec = cpu_decode_baseline(path, prompt, gold["config"]) if cpu else None
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
            "tokens_match_reference_cpu_loop": ids == gold["tokens"], "model_write_s": round(t_write, 1),
            "cpu_baseline": cpu_dec}


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


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            return next(line.split(":", 1)[1].strip() for line in f if line.startswith("model name"))
    except (OSError, StopIteration):
        return ""


def _cpu_time(run, n_copies: int, budget_s: float, min_calls: int = 5) -> tuple[float, int]:
    """Median seconds per call of run(copy index) over about budget_s, after two warm-up calls."""
    for i in range(2):
        run(i % n_copies)
    times = []
    t_end = time.perf_counter() + budget_s
    i = 0
    while time.perf_counter() < t_end or len(times) < min_calls:
        t = time.perf_counter()
        run(i % n_copies)
        times.append(time.perf_counter() - t)
        i += 1
    return float(np.median(times)), len(times)


def cpu_baseline(budget_s: float) -> dict | None:
    """The reference's own kernels (oracle/_ref: its widest table on this CPU, OpenMP) on bounded
    samples of the GPU cases: the headline Q4_0 GEMV on all allowed cores (the line's value) and,
    on one core and on all of them, Q4_0 at 8192x2048 and 14336x4096, Q8_0 at both Llama-3.2-1B
    FFN orientations, FP16 and BF16 trans_b GEMVs at 4096x4096.  Weights rotate through more than
    512 MiB of host copies (per case) so the host caches cannot hold them.  Without oracle/_ref
    (no reference sources where the library was built): the oracle's scalar C restatement of the
    headline on one core."""
    from oracle import oracle as o  # the checker/baseline leg only
    cores = len(os.sched_getaffinity(0))
    R = o.ref()
    model = _cpu_model()
    rng = np.random.default_rng(0)
    if R is None:
        N, K = 8192, 2048
        x = rng.standard_normal(K, dtype=np.float32)
        w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
        wq = o.quantize_q4_0(w)
        y = np.zeros(N, np.float32)
        run = lambda c: o.lib().smko_gemv_q4_0(N, K, x.ctypes.data_as(o._f32p), wq.ctypes.data_as(o._u8p),
                                               y.ctypes.data_as(o._f32p))
        med, n = _cpu_time(run, 1, budget_s)
        return {"value": wq.nbytes / med / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{n} gemv_q4_0 calls 8192x2048 (median {med * 1e6:.1f} us), oracle C restatement "
                          f"(scalar), no rotation; {model}"}
    isa = o.ref_best_isa()
    path = R.ref_q8_0_path(o.ISA[isa]).decode()
    share = budget_s / 16  # per (case, thread count); the headline on all cores gets a quarter

    def gemv_case(fmt: str, N: int, K: int, threads: int, secs: float) -> dict:
        x = rng.standard_normal(K, dtype=np.float32)
        w = rng.standard_normal((N, K), dtype=np.float32)
        w *= np.float32(0.02)
        y = np.zeros(N, np.float32)
        xp, yp = x.ctypes.data_as(o._f32p), y.ctypes.data_as(o._f32p)
        if fmt in ("q4_0", "q8_0"):
            wq = (o.quantize_q4_0 if fmt == "q4_0" else o.quantize_q8_0)(w)
            fn = R.ref_gemv_q4_0 if fmt == "q4_0" else R.ref_gemv_q8_0
            run1 = lambda c: fn(o.ISA[isa], N, K, xp, c.ctypes.data_as(o._u8p), yp)
        else:
            if fmt == "f16":
                xb, wq = x.astype(np.float16).view(np.uint16), w.astype(np.float16).view(np.uint16)
                fn = R.ref_sgemm_f16
            else:  # bf16 by truncation, as the GPU case
                xb, wq = (x.view(np.uint32) >> 16).astype(np.uint16), (w.view(np.uint32) >> 16).astype(np.uint16)
                fn = R.ref_sgemm_bf16
            run1 = lambda c: fn(o.ISA[isa], 1, 1, N, K, 1.0, xb.ctypes.data, K, c.ctypes.data, K, 0.0, yp, N)
        del w
        copies = [wq] + [wq.copy() for _ in range(math.ceil(ROTATE_BYTES / wq.nbytes))]
        R.ref_set_num_threads(threads)
        med, n = _cpu_time(lambda i: run1(copies[i]), len(copies), secs)
        return {"GBps": round(wq.nbytes / med / 1e9, 2), "us": round(med * 1e6, 2), "calls": n,
                "weight_bytes": int(wq.nbytes), "copies": len(copies)}

    head = gemv_case("q4_0", 8192, 2048, cores, 4 * share)
    cases = {}
    for fmt, N, K in (("q4_0", 8192, 2048), ("q4_0", 14336, 4096), ("q8_0", 8192, 2048), ("q8_0", 2048, 8192),
                      ("f16", 4096, 4096), ("bf16", 4096, 4096)):
        key = f"{fmt}_{N}x{K}"
        cases[key] = {"one_core": gemv_case(fmt, N, K, 1, share)}
        cases[key]["all_cores"] = head if key == "q4_0_8192x2048" else gemv_case(fmt, N, K, cores, share)
    R.ref_set_num_threads(cores)
    return {"value": head["GBps"], "unit": "GB/s", "cores": cores, "kind": "reference",
            "sample": f"{head['calls']} gemv_q4_0 calls 8192x2048 (median {head['us']:.1f} us) over "
                      f"{head['copies']} rotated host copies ({head['copies'] * head['weight_bytes'] / 2 ** 20:.0f} "
                      f"MiB); {isa} table, {path} inner loop; {model}",
            "isa": isa, "q8_0_path": path, "cpu": model, "cases": cases}


def cpu_decode_baseline(path: str, prompt: list[int], config: dict, n_steps: int = 24,
                        n_prompt: int = 8) -> dict | None:
    """Decode tok/s of the reference's own kernels (oracle/_ref) through the example's loop
    (oracle/llama_ref.Decoder, "reference" kind: llama.py:414-505 with gemv_q4_0, sgemm, softmax_row
    and silu from the reference's table) on the same GGUF model as the GPU decode: n_prompt tokens
    of the prompt, then n_steps timed greedy steps, on all allowed cores and on one."""
    from oracle import llama_ref as lr  # the checker/baseline leg only
    from oracle import oracle as o
    from simd_ml_kernels.gguf import GGUF

    R = o.ref()
    if R is None:
        return None
    cores = len(os.sched_getaffinity(0))
    cfg = lr.Cfg.from_config(config)
    g = GGUF(path)
    W = {"token_embd": g.tensors["token_embd.weight"].data}
    for i in range(cfg.n_layers):
        for nm in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"):
            W[f"{i}.{nm}"] = g.tensors[f"blk.{i}.{nm}.weight"].data
    out = {}
    for threads, key in ((cores, "all_cores"), (1, "one_core")):
        R.ref_set_num_threads(threads)
        dec = lr.Decoder(cfg, W, lr.Q4_0, "reference")
        dec.reset(n_prompt + n_steps + 1)
        logits = None
        for t in prompt[:n_prompt]:
            logits = dec.step(t)
        steps = n_steps if threads > 1 else max(4, n_steps // 4)
        t0 = time.perf_counter()
        for _ in range(steps):
            logits = dec.step(int(np.argmax(logits)))
        dt = time.perf_counter() - t0
        out[key] = {"tok_s": round(steps / dt, 2), "ms_per_token": round(1e3 * dt / steps, 2), "steps": steps,
                    "threads": threads}
    R.ref_set_num_threads(cores)
    out["loop"] = "oracle/llama_ref.Decoder 'reference' kind (the example's numpy loop on oracle/_ref kernels)"
    return out


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
    if args.cases == "shapes":
        out = {}
        for spec in args.shape or [f"{f}:{n}x{k}" for f in ("q4_0", "q8_0") for n, k in ((14336, 4096), (4096, 14336))]:
            fmt, dims = spec.split(":")
            N, K = (int(v) for v in dims.lower().split("x"))
            if fmt in BB:
                out[f"{fmt}_{N}x{K}"] = quant_case(dev, fmt, N, K, 3, args.steps, args.warmup, args.mode)
            elif fmt in ("f16", "bf16"):
                out[f"{fmt}_{N}x{K}"] = lowp_case(dev, fmt, N, K, 2, args.steps, args.warmup, args.mode)
            else:
                raise SystemExit(f"--shape {spec}: format must be one of q4_0, q8_0, f16, bf16")
        print(json.dumps({"shapes": out}))
        return 0
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
    decode = decode_case(cpu=not args.no_cpu) if args.cases == "all" else None
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
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        if out["cpu_baseline"] is not None and decode is not None:
            out["cpu_baseline"]["decode"] = decode.pop("cpu_baseline", None)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
