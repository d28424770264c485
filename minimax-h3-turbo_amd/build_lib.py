"""Build the h3k HIP library for gfx950: csrc/*.hip -> h3turbo_amd/libh3k.so (in-tree).

    python minimax-h3-turbo_amd/build_lib.py [-j N] [--verbose]

hipcc cross-compiles without a GPU.  Flags that matter for the numerics: -ffp-contract=off (the epilogue's
separate roundings), correctly rounded fp32 division, no fast-math; packed fp32 instructions are disabled.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "h3turbo_amd", "libh3k.so")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm 7.x needed to build the h3k library)")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in p.stdout.splitlines() if "packed-fp32-ops" not in line)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def guard_weight_loads(obj: str) -> None:
    """Fail the build when the compiler touched an in-flight inline-assembly weight register (asm_guard.py)."""
    sys.path.insert(0, HERE)
    import asm_guard

    if not asm_guard.available():
        raise RuntimeError("llvm-objcopy / clang-offload-bundler / llvm-objdump not found under /opt/rocm/llvm/bin: "
                           "the weight-register guard of h3k_gemm_w8p.o cannot run")
    bad = asm_guard.check_object(obj)
    if bad:
        raise RuntimeError("h3k_gemm_w8p.o: the compiler touches asynchronous weight registers in flight:\n  " +
                           "\n  ".join(bad[:10]))


def build(jobs: int = 4, verbose: bool = False) -> str:
    cc = hipcc()
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = [os.path.join(BUILD, s[:-4] + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = [ex.submit(_run, [cc, *FLAGS, "-c", os.path.join(CSRC, s), "-o", o], verbose) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    guard_weight_loads(os.path.join(BUILD, "h3k_gemm_w8p.o"))
    tmp = OUT + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.verbose))
    sys.exit(0)
