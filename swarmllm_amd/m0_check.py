"""The M0 invariant of csrc/lds_copy.h, checked over the AMD assembly of the
library's own build.

dma16 / dma4 set M0 to the LDS destination right before each
global_load_lds and declare M0 clobbered; the compiler does not track M0
through inline assembly, so a kernel that copies this way must not read M0
anywhere else (an instruction reading it would see a copy's LDS address, or
the compiler's value would be lost under a copy). The check disassembles the
gfx950 code object of every built object, and in every function that holds
a global_load_lds copy it requires:
  - each copy is preceded by its own `s_mov_b32 m0, ...` and `s_nop 0`
    (the form dma16 / dma4 emit);
  - no other instruction reads M0: neither as an explicit source operand nor
    implicitly (message sends, indexed register moves, interpolation, GWS,
    append / consume, addtid LDS access, the other LDS-direct loads).
build_library runs it after every build and fails the build on a violation.
"""
from __future__ import annotations

import glob
import os
import re
import subprocess
import tempfile
from typing import Dict, List, Tuple

LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

# instructions that read M0 without naming it
IMPLICIT_READERS = ("s_sendmsg", "s_ttracedata", "v_movrel", "s_movrel", "v_interp", "ds_gws", "ds_append",
                    "ds_consume", "ds_read_addtid", "ds_write_addtid", "s_set_gpr_idx", "s_cbranch_g_fork",
                    "buffer_load_lds", "buffer_store_lds", "scratch_load_lds")
COPY = re.compile(r"^global_load_lds_")
FUNC = re.compile(r"^[0-9a-fA-F]+ <(.+)>:$")

Inst = Tuple[str, List[str]]


def parse(disasm: str) -> Dict[str, List[Inst]]:
    """llvm-objdump -d text -> {function: [(mnemonic, operands)]}."""
    funcs: Dict[str, List[Inst]] = {}
    cur = None
    for line in disasm.splitlines():
        m = FUNC.match(line.strip())
        if m:
            cur = m.group(1)
            funcs[cur] = []
            continue
        if cur is None:
            continue
        text = line.split("//", 1)[0].strip()
        if not text or text.endswith(":"):
            continue
        parts = text.split(None, 1)
        ops = [o.strip() for o in parts[1].split(",")] if len(parts) > 1 else []
        funcs[cur].append((parts[0], ops))
    return funcs


def _is_lds_buffer_load(mn: str, ops: List[str]) -> bool:
    # buffer_load_* ... lds: the other LDS-direct form, which reads M0
    return mn.startswith("buffer_load") and any(o.split()[-1] == "lds" for o in ops if o)


def _reads_m0(mn: str, ops: List[str]) -> bool:
    if mn.startswith(IMPLICIT_READERS) or _is_lds_buffer_load(mn, ops):
        return True
    srcs = ops[1:] if ops else []
    return any(re.search(r"\bm0\b", o) for o in srcs)


def violations(disasm: str) -> List[str]:
    """The breaches of the invariant in one object's disassembly."""
    out = []
    for name, insts in parse(disasm).items():
        if not any(COPY.match(mn) for mn, _ in insts):
            continue
        for i, (mn, ops) in enumerate(insts):
            if COPY.match(mn):
                ok = (i >= 2 and insts[i - 1][0] == "s_nop" and insts[i - 2][0] == "s_mov_b32"
                      and insts[i - 2][1][:1] == ["m0"])
                if not ok:
                    out.append(f"{name}: instruction {i} ({mn}) is not preceded by its own s_mov_b32 m0 / s_nop 0")
            elif _reads_m0(mn, ops):
                out.append(f"{name}: instruction {i} reads M0: {mn} {', '.join(ops)}")
    return out


def disassemble(obj: str) -> str:
    """The gfx950 device code of a hipcc-built object, as llvm-objdump text."""
    with tempfile.TemporaryDirectory() as t:
        fb, co = os.path.join(t, "fb.bin"), os.path.join(t, "x.co")
        subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fb}", obj, os.path.join(t, "o.o")],
                       check=True, capture_output=True)
        subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={fb}",
                        f"--targets={TARGET}", f"--output={co}"], check=True, capture_output=True)
        res = subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", co], check=True, capture_output=True,
                             text=True)
        return res.stdout


def has_device_code(obj: str) -> bool:
    res = subprocess.run([f"{LLVM}/llvm-readelf", "-S", obj], capture_output=True, text=True)
    return ".hip_fatbin" in res.stdout


def check_objects(objs: List[str]) -> Tuple[List[str], int]:
    """(violations, number of functions that copy through M0) over objects."""
    found, copying = [], 0
    for obj in objs:
        if not has_device_code(obj):
            continue
        text = disassemble(obj)
        copying += sum(1 for insts in parse(text).values() if any(COPY.match(mn) for mn, _ in insts))
        found += [f"{os.path.basename(obj)}: {v}" for v in violations(text)]
    return found, copying


def check_build(build_dir: str) -> int:
    """Raise if any built object breaks the invariant; the number of
    copying functions otherwise."""
    objs = sorted(glob.glob(os.path.join(build_dir, "*.o")))
    found, copying = check_objects(objs)
    if found:
        raise RuntimeError("M0 invariant of lds_copy.h broken:\n  " + "\n  ".join(found))
    return copying
