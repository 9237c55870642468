"""Build ``lib/libhcp_ring_amd.so`` from ``csrc/*.hip`` with hipcc for gfx950.

Every translation unit is compiled in-tree (the shared library travels with the
repository to the GPU box); objects go to ``_build/``.  Objects whose kernels use the
LDS DMA helper are disassembled and checked: M0 may only appear in that helper's own
instruction sequence (the compiler does not track the helper's M0 write).  Usage::

    python hetero-cp-ringattn_amd/build.py [-j N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import re
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libhcp_ring_amd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(HERE, '..', 'include')}",
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


LLVM_BIN = os.environ.get("HCP_LLVM_BIN", "/opt/rocm/llvm/bin")
# the helper's scalar operand: any SGPR, including the named ones the allocator may
# hand out under pressure (vcc_lo / vcc_hi)
M0_SEQ = re.compile(r"^s_mov_b32 m0, (s\d+|vcc_lo|vcc_hi)$")
# instructions that read or write M0 without naming it
M0_IMPLICIT = re.compile(r"^(v_movrel|s_movrel|s_set_gpr_idx|s_sendmsg|ds_gws|ds_\w*addtid|v_interp|"
                         r"lds_param_load|lds_direct_load|global_load_lds|scratch_load_lds|s_ttracedata)")


def device_asm(obj: str) -> list[str]:
    """Disassembly (instruction text only) of the gfx950 code object inside `obj`."""
    with tempfile.TemporaryDirectory() as tmp:
        fat, co = os.path.join(tmp, "fatbin"), os.path.join(tmp, "code.co")
        subprocess.run([os.path.join(LLVM_BIN, "llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", obj,
                        os.path.join(tmp, "scratch.o")], check=True, capture_output=True)
        subprocess.run([os.path.join(LLVM_BIN, "clang-offload-bundler"), "--unbundle", "--type=o",
                        f"--targets=hipv4-amdgcn-amd-amdhsa--{ARCH}", f"--input={fat}", f"--output={co}"],
                       check=True, capture_output=True)
        out = subprocess.run([os.path.join(LLVM_BIN, "llvm-objdump"), "-d", f"--mcpu={ARCH}", co],
                             check=True, capture_output=True, text=True).stdout
    lines = []
    for raw in out.splitlines():
        text = raw.split("//", 1)[0].strip()
        if text and not text.endswith(">:") and raw.startswith("\t"):
            lines.append(text)
    return lines


def check_m0(obj: str) -> int:
    """The LDS DMA helper (csrc/lds_dma.hpp) sets M0 inside inline asm, which the
    compiler does not track: it is correct only while nothing else in the code object
    reads or writes M0.  Every M0 access must be the helper's own three-instruction
    sequence (s_mov_b32 m0, sN; s_nop 0; buffer_load_dwordx4 ... lds); raises otherwise.
    Returns the number of sequences found."""
    return scan_m0(device_asm(obj), os.path.basename(obj))


def scan_m0(ins: list[str], name: str = "code object") -> int:
    """check_m0 on a list of instructions."""
    seqs = 0
    i = 0
    while i < len(ins):
        t = ins[i]
        if M0_IMPLICIT.match(t):
            raise RuntimeError(f"{name}: instruction that uses M0 implicitly: {t}")
        if re.search(r"\bm0\b", t) or " lds" in t and t.startswith("buffer_load"):
            ok = (M0_SEQ.match(t) is not None and i + 2 < len(ins) and ins[i + 1] == "s_nop 0" and
                  ins[i + 2].startswith("buffer_load_dwordx4") and ins[i + 2].endswith(" lds"))
            if not ok:
                ctx = "\n  ".join(ins[max(0, i - 3):i + 4])
                raise RuntimeError(f"{name}: M0 used outside the LDS DMA sequence:\n  {ctx}")
            seqs += 1
            i += 3
            continue
        i += 1
    return seqs


def build(jobs: int | None = None) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = jobs or min(8, len(srcs))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    for src, obj in zip(srcs, objs):
        if "lds_dma.hpp" in open(src).read():
            check_m0(obj)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    args = ap.parse_args()
    print(build(args.j))
