#!/usr/bin/env python3
"""Build check of the library's gfx950 code objects (run by the Makefile after linking).

For every object under build/: take the gfx950 code object out of its offload bundle,
disassemble it and fail when

  * any packed-FP32 arithmetic instruction (the add, mul and fma forms) appears: every HIP
    file is compiled with the packed-FP32 target feature disabled, and this confirms the
    compiler honoured it; or
  * any kernel has a private segment (scratch): register spills or stack arrays, which cost
    memory traffic on every launch.

Uses the ROCm LLVM tools only (objcopy from binutils for the bundle section).  Exit status 0
when clean; the report names each offending kernel.
"""

from __future__ import annotations

import os
import re
import subprocess
import sys
import tempfile

LLVM = os.environ.get("ROCM_LLVM", "/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
PACKED_F32 = re.compile(r"\bv_pk_(add|mul|fma)_f32\b")


def code_object(obj: str, tmp: str) -> str | None:
    """Path of the gfx950 code object of one compiled .o (None: no device code in it)."""
    fat = os.path.join(tmp, os.path.basename(obj) + ".fatbin")
    co = os.path.join(tmp, os.path.basename(obj) + ".co")
    r = subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", obj, fat], capture_output=True)
    if r.returncode != 0 or not os.path.exists(fat) or os.path.getsize(fat) == 0:
        return None
    r = subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o", f"--input={fat}",
                        f"--targets={TARGET}", f"--output={co}"], capture_output=True)
    return co if r.returncode == 0 and os.path.getsize(co) > 0 else None


def scratch_kernels(co: str) -> list[tuple[str, int]]:
    notes = subprocess.run([os.path.join(LLVM, "llvm-readelf"), "--notes", co], capture_output=True, text=True,
                           check=True).stdout
    out = []
    for block in notes.split("- .agpr_count")[1:]:
        name = re.search(r"\.name:\s+(\S+)", block)
        size = re.search(r"\.private_segment_fixed_size:\s+(\d+)", block)
        if name and size and int(size.group(1)) > 0:
            out.append((name.group(1), int(size.group(1))))
    return out


def packed_f32(co: str) -> int:
    text = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", co], capture_output=True, text=True,
                          check=True).stdout
    return len(PACKED_F32.findall(text))


def demangle(names: list[str]) -> list[str]:
    r = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True)
    return r.stdout.splitlines() if r.returncode == 0 else names


def main(build_dir: str) -> int:
    objs = sorted(os.path.join(build_dir, f) for f in os.listdir(build_dir) if f.endswith(".o"))
    bad = 0
    kernels = 0
    with tempfile.TemporaryDirectory() as tmp:
        for obj in objs:
            co = code_object(obj, tmp)
            if co is None:
                continue
            n_pk = packed_f32(co)
            if n_pk:
                print(f"check_objects: {os.path.basename(obj)}: {n_pk} packed-FP32 instructions", file=sys.stderr)
                bad += 1
            spills = scratch_kernels(co)
            for (mangled, size), pretty in zip(spills, demangle([m for m, _ in spills])):
                print(f"check_objects: {os.path.basename(obj)}: {size} bytes of scratch per lane in {pretty}",
                      file=sys.stderr)
                bad += 1
            kernels += subprocess.run([os.path.join(LLVM, "llvm-readelf"), "--notes", co], capture_output=True,
                                      text=True).stdout.count(".private_segment_fixed_size")
    print(f"check_objects: {len(objs)} objects, {kernels} kernels, "
          f"{'clean' if not bad else f'{bad} problem(s)'} (no packed FP32, no scratch)")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1] if len(sys.argv) > 1 else os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                                      "build")))
