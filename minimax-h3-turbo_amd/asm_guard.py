"""Build-time guard for the large-shape GEMM's asynchronous weight loads (csrc/h3k_gemm_w8p.hip).

The kernel loads its weight fragments with inline-assembly buffer loads that the compiler's wait insertion cannot
see: the compiler treats the destination registers as written when the load issues, while the data lands hundreds
of cycles later (the kernel's explicit waits cover the MFMAs that read them).  That is only correct while nothing
else touches those registers in flight.  This check disassembles the gfx950 code object of h3k_gemm_w8p.o and
follows each such load in text order: the first later instruction that touches any of its registers -- before a
vmcnt(0) wait has made the data land -- must be an MFMA reading them or another weight load writing them.  A copy,
a spill or a reuse of the registers fails the build.

    python minimax-h3-turbo_amd/asm_guard.py path/to/h3k_gemm_w8p.o
"""
from __future__ import annotations

import os
import re
import subprocess
import sys
import tempfile
from typing import List, Set, Tuple

LLVM = "/opt/rocm/llvm/bin"
KERNEL = "_ZN3h3k3w8p15gemm_w8p_kernel"


def _regs(tok: str) -> Set[int]:
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _is_weight_load(line: str) -> bool:
    # the kernel's only register-returning buffer loads (the activation loads go to LDS: "lds")
    return line.startswith("buffer_load_dwordx4") and not line.endswith(" lds") and " offen" in line


def _touched(line: str) -> Tuple[str, Set[int]]:
    op, _, rest = line.partition(" ")
    out: Set[int] = set()
    for t in rest.split(","):
        t = t.strip().split(" ")[0]
        out |= _regs(t)
    return op, out


def kernels_of_disassembly(text: str) -> List[Tuple[str, List[str]]]:
    """(symbol, instructions) of each gemm_w8p kernel in llvm-objdump -d output."""
    out: List[Tuple[str, List[str]]] = []
    cur = None
    for raw in text.splitlines():
        m = re.match(r"^[0-9a-f]+ <(\S+)>:", raw)
        if m:
            cur = (m.group(1), []) if m.group(1).startswith(KERNEL) else None
            if cur:
                out.append(cur)
            continue
        if cur is None:
            continue
        line = raw.split("//")[0].strip()
        if line and not line.endswith(":"):
            cur[1].append(line)
    return out


def violations(kernels: List[Tuple[str, List[str]]]) -> List[str]:
    bad: List[str] = []
    for name, lines in kernels:
        loads = 0
        for i, line in enumerate(lines):
            if not _is_weight_load(line):
                continue
            loads += 1
            regs = _regs(line.split()[1].rstrip(","))
            for later in lines[i + 1:]:
                if later.startswith("s_waitcnt") and "vmcnt(0)" in later:
                    break
                op, t = _touched(later)
                if not (t & regs):
                    continue
                if not (op.startswith("v_mfma") or _is_weight_load(later)):
                    bad.append(f"{name}: `{line}` then `{later}`")
                break
        if loads == 0:
            bad.append(f"{name}: no weight loads found (the guard no longer matches the kernel)")
    if not kernels:
        bad.append("no gemm_w8p kernels in the code object")
    return bad


def check_object(obj: str) -> List[str]:
    """Violations in the gfx950 code object of a hipcc -c object file."""
    with tempfile.TemporaryDirectory() as d:
        fat, co = os.path.join(d, "fat.bin"), os.path.join(d, "k.co")
        subprocess.run([os.path.join(LLVM, "llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", obj, os.path.join(d, "x.o")],
                       check=True, capture_output=True)
        subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--type=o", f"--input={fat}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}", "--unbundle"],
                       check=True, capture_output=True)
        dis = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--mcpu=gfx950", co], check=True,
                             capture_output=True, text=True).stdout
    return violations(kernels_of_disassembly(dis))


def available() -> bool:
    return all(os.path.exists(os.path.join(LLVM, t)) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"))


if __name__ == "__main__":
    bad = check_object(sys.argv[1])
    for b in bad:
        print(b)
    print(f"{len(bad)} violation(s)")
    sys.exit(1 if bad else 0)
