"""``python -m simd_ml_kernels selftest | info``: a one-command check of the device kernels.

Mirrors the reference's ``selftest`` command (python/simd_ml_kernels/_cli.py:324-348): every
in-scope kernel of the single "gfx950" table runs on small inputs and is compared with a float64
value computed here, against the error bound the reference documents for it; one line per check
(PASS / FAIL, the worst error as a fraction of its bound), then "selftest: passed" or "FAILED"
and exit status 0 / 1.  A failing or raising check is reported and the others still run.

The float64 values come from numpy on the same operands the kernel sees (for the quantized
GEMVs: W's blocks and x's Q8 quants, as the reference's checker takes them); no part of the test
infrastructure is imported.  Needs a gfx950 device: without one every check fails loudly.
"""

from __future__ import annotations

import argparse
import sys
from typing import Callable

import numpy as np

U32 = 2.0 ** -24  # unit roundoff of float32


def _sk():
    import simd_ml_kernels as sk
    return sk


# ─── float64 values of the quantized products ──────────────────────────────


def _scales_f16(blocks: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(blocks[:, :, :2]).view("<f2")[:, :, 0].astype(np.float64)


def _q8_blocks(wq: np.ndarray, n: int, k: int):
    b = np.ascontiguousarray(wq).reshape(n, k // 32, 34)
    return _scales_f16(b), np.ascontiguousarray(b[:, :, 2:]).view(np.int8).astype(np.int64)


def _q4_blocks(wq: np.ndarray, n: int, k: int):
    b = np.ascontiguousarray(wq).reshape(n, k // 32, 18)
    nib = b[:, :, 2:]
    q = np.concatenate([nib & 0x0F, nib >> 4], axis=2).astype(np.int64) - 8  # value j low, 16 + j high
    return _scales_f16(b), q


def _x_q8(x: np.ndarray):
    """x's Q8 blocks as the kernels form them: fp32 d = amax / 127, quants round(x * (1/d)) half
    away from zero (0 for an all-zero block), the scale kept in fp32."""
    xb = x.astype(np.float32).reshape(-1, 32)
    d = (np.abs(xb).max(axis=1) / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    p = (xb * inv[:, None]).astype(np.float32).astype(np.float64)  # one fp32 product, then exact
    q = np.sign(p) * np.floor(np.abs(p) + 0.5)
    return d.astype(np.float64), q.astype(np.int64)


def _quant_reference(x: np.ndarray, dw: np.ndarray, qw: np.ndarray):
    """Exact (float64) y and the bound's magnitude sum_b |dw dx| sum_i |qw qx| per row."""
    dx, qx = _x_q8(x)
    sc = dw * dx[None, :]
    prod = qw * qx[None, :, :]
    return ((prod.sum(axis=2) * sc).sum(axis=1), (np.abs(prod).sum(axis=2) * np.abs(sc)).sum(axis=1))


def _gemv_check(fmt: str):
    shapes = [(1, 32), (7, 64), (9, 96), (17, 320), (33, 4096), (65, 14336)]

    def check():
        sk = _sk()
        rng = np.random.default_rng(5 if fmt == "q4_0" else 4)
        worst, where = 0.0, ""
        for n, k in shapes:
            w = rng.standard_normal((n, k)).astype(np.float32)
            x = rng.standard_normal(k).astype(np.float32)
            if fmt == "q4_0":
                wq = sk.quantize_q4_0(w)
                dw, qw = _q4_blocks(wq, n, k)
                y = sk.gemv_q4_0(x, wq, n, k)
            else:
                wq = sk.quantize_q8_0(w)
                dw, qw = _q8_blocks(wq, n, k)
                y = sk.gemv_q8_0(x, wq, n, k)
            ref, mag = _quant_reference(x, dw, qw)
            r = float(np.max(np.abs(y.astype(np.float64) - ref) / (2 * (k // 32 + 4) * U32 * mag + 1e-300)))
            if r > worst:
                worst, where = r, f"N={n} K={k}"
        sign = "(qw-8)" if fmt == "q4_0" else "qw"
        return worst, f"max err / (2*(K/32+4)*u*sum|dw dx||{sign} qx|), worst at {where}"
    return check


# ─── float32 / float16 / bfloat16 products ─────────────────────────────────


def _as_f16(a: np.ndarray):
    h = a.astype(np.float16)
    return h, h.astype(np.float64)


def _as_bf16(a: np.ndarray):
    bits = (a.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    return bits, (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _as_f32(a: np.ndarray):
    a = a.astype(np.float32)
    return a, a.astype(np.float64)


def _gemm_check(fn_name: str, cast: Callable):
    # Decode GEMVs (one row, trans_b) and a few small products; K past the 64-lane kernel's
    # threshold and odd K included.
    cases = [(1, 64, 4099), (1, 4096, 300), (1, 300, 4096), (1, 65, 14336), (4, 33, 1027), (8, 45, 133)]

    def check():
        sk = _sk()
        fn = getattr(sk, fn_name)
        rng = np.random.default_rng(7)
        worst, where = 0.0, ""
        for m, n, k in cases:
            a, a64 = cast(rng.standard_normal((m, k)))
            b, b64 = cast(rng.standard_normal((n, k)))
            c = np.asarray(fn(a, b, trans_b=True)).astype(np.float64).reshape(m, n)
            ref, mag = a64 @ b64.T, np.abs(a64) @ np.abs(b64).T
            r = float(np.max(np.abs(c - ref) / (2 * (k + 2) * U32 * mag + 1e-300)))
            if r > worst:
                worst, where = r, f"{m}x{n}x{k}"
        return worst, f"max err / (2*(K+2)*u*|A||B|^T), trans_b, worst at {where}"
    return check


# ─── elementwise steps ─────────────────────────────────────────────────────


def _silu_check():
    sk = _sk()
    rng = np.random.default_rng(1)
    xs = [np.linspace(-200.0, 200.0, 20_001).astype(np.float32)]
    xs += [rng.uniform(-200.0, 200.0, n).astype(np.float32) for n in (1, 7, 9, 15, 4099)]
    worst = 0.0
    for x in xs:
        x64 = x.astype(np.float64)
        with np.errstate(over="ignore"):
            ref = x64 / (1.0 + np.exp(-x64))
        err = np.abs(sk.silu(x).astype(np.float64) - ref)
        worst = max(worst, float(np.max(err / (1e-35 + 1e-6 * np.abs(ref)))))
    return worst, "max err / (1e-35 + 1e-6*|ref|) on [-200, 200]"


def _softmax_check():
    sk = _sk()
    rng = np.random.default_rng(2)
    worst = 0.0
    for shape in [(1,), (7,), (8,), (3, 9), (4, 1000), (2, 4099)]:
        x = (3.0 * rng.standard_normal(shape)).astype(np.float32)
        x64 = x.astype(np.float64)
        e = np.exp(x64 - x64.max(axis=-1, keepdims=True))
        ref = e / e.sum(axis=-1, keepdims=True)
        worst = max(worst, float(np.max(np.abs(sk.softmax(x).astype(np.float64) - ref)) / 1e-6))
    return worst, "max abs err / 1e-6"


def _rms_norm_check():
    sk = _sk()
    rng = np.random.default_rng(3)
    worst = 0.0
    for n in (1, 7, 64, 2048, 4099):
        x = rng.standard_normal((3, n)).astype(np.float32)
        w = rng.standard_normal(n).astype(np.float32)
        x64 = x.astype(np.float64)
        ref = w.astype(np.float64) * x64 / np.sqrt((x64 * x64).mean(axis=-1, keepdims=True) + 1e-5)
        err = np.abs(sk.rms_norm(x, w, 1e-5).astype(np.float64) - ref)
        worst = max(worst, float(np.max(err / (1e-6 + 1e-5 * np.abs(ref)))))
    return worst, "max err / (1e-6 + 1e-5*|ref|)"


def _rope_check():
    sk = _sk()
    rng = np.random.default_rng(6)
    worst = 0.0
    for heads, hd in ((1, 4), (8, 64), (4, 128)):
        x = rng.standard_normal((heads, hd)).astype(np.float32)
        ang = rng.uniform(-np.pi, np.pi, hd // 2)
        for interleaved in (True, False):
            half_c, half_s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
            # Pair i turns by angle i in both layouts; the tables are [head_dim] with equal halves.
            c, s = np.concatenate([half_c, half_c]), np.concatenate([half_s, half_s])
            if interleaved:
                x64 = x.astype(np.float64)
                a, b = x64[:, 0::2], x64[:, 1::2]
                ref = np.empty_like(x64)
                ref[:, 0::2] = a * half_c - b * half_s
                ref[:, 1::2] = b * half_c + a * half_s
            else:
                x64 = x.astype(np.float64)
                lo, hi = x64[:, :hd // 2], x64[:, hd // 2:]
                ref = np.concatenate([lo * half_c - hi * half_s, hi * half_c + lo * half_s], axis=1)
            y = sk.rope(x, c, s, interleaved).astype(np.float64)
            mag = np.abs(x64).max(axis=1, keepdims=True)
            worst = max(worst, float(np.max(np.abs(y - ref) / (4 * U32 * mag + 1e-300))))
    return worst, "max err / (4*u*max|x|), interleaved and half-split"


def _xquant_check():
    from simd_ml_kernels import abi
    import ctypes
    counts = (ctypes.c_uint * 2)()
    abi.call("smk_selfcheck_q8", counts)
    bad = int(counts[0]) + int(counts[1])
    return float(bad), f"x quantizer forms vs IEEE divisions: {counts[0]} scale, {counts[1]} rounding mismatches"


def selftest_checks() -> list[tuple[str, Callable[[], tuple]]]:
    return [
        ("x quantizer", _xquant_check),
        ("gemv_q4_0", _gemv_check("q4_0")),
        ("gemv_q8_0", _gemv_check("q8_0")),
        ("sgemm tb", _gemm_check("sgemm", _as_f32)),
        ("sgemm_f16 tb", _gemm_check("sgemm_f16", _as_f16)),
        ("sgemm_bf16 tb", _gemm_check("sgemm_bf16", _as_bf16)),
        ("silu", _silu_check),
        ("softmax", _softmax_check),
        ("rms_norm", _rms_norm_check),
        ("rope", _rope_check),
    ]


def cmd_selftest() -> int:
    sk = _sk()
    info = sk.build_info()
    print(f"simd_ml_kernels {info.get('version', '?')} ({info.get('library', '?')}) on "
          f"{info.get('gemv_device') or 'no device'}, kernel table {sk.detected_isa()}")
    print(f" [{sk.detected_isa()}]")
    failed = 0
    for name, check in selftest_checks():
        try:
            worst, detail = check()
            ok = worst <= (0.0 if name == "x quantizer" else 1.0)
        except Exception as exc:  # report every failure, keep going
            worst, ok, detail = float("nan"), False, f"{type(exc).__name__}: {exc}"
        failed += not ok
        print(f"  {'PASS' if ok else 'FAIL'}  {name:<14} {worst:8.3f}  {detail}", flush=True)
    print("selftest:", "FAILED" if failed else "passed")
    return 1 if failed else 0


def cmd_info() -> int:
    sk = _sk()
    for k, v in sorted(sk.build_info().items()):
        print(f"{k}: {v}")
    return 0


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(prog="python -m simd_ml_kernels")
    p.add_argument("command", choices=["selftest", "info"])
    args = p.parse_args(argv)
    return cmd_selftest() if args.command == "selftest" else cmd_info()


if __name__ == "__main__":
    sys.exit(main())
