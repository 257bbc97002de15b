"""Builds the HIP library reels_amd/lib/libreels_hip.so for gfx950 with hipcc (in-tree).

Run as ``python -m reels_amd.build`` or through ``__graft_entry__.build()``. Every call
recompiles every source; objects go to reels_amd/lib/obj/ and are linked into one shared library.
The sources with LDS-DMA copies are also compiled to assembly and checked for a hazard the
compiler does not guard around inline asm (lds_dma_hazards); the build fails on one.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import re
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libreels_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in device code (the host pass ignores the feature).
# No fast-math: the pack kernel relies on IEEE division and preserved f32 denormals.
DEVICE_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: str, obj: str) -> None:
    cmd = [HIPCC, *DEVICE_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def _sregs(spec: str) -> set:
    out = set()
    for m in re.finditer(r"s\[(\d+):(\d+)\]|\bs(\d+)\b|\b(m0)\b", spec):
        if m.group(4):
            out.add("m0")
        elif m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def lds_dma_hazards(asm_text: str) -> list:
    """LDS-DMA copies (``buffer_load_dwordx4 ... lds``, issued through inline asm) whose SGPR
    operands or M0 were written by a VALU instruction fewer than five wait states earlier. On
    gfx950 a VMEM instruction needs five wait states after a VALU write of an SGPR it reads; the
    compiler inserts them for its own instructions but not around inline asm, and it emits such
    writes (v_readlane_b32) when it reloads spilled SGPRs. Returns (function, line, writer)."""
    hits, insts, func = [], [], "?"
    for i, line in enumerate(asm_text.splitlines()):
        s = line.strip()
        m = re.match(r"^(_Z\w+):", s)
        if m:
            func, insts = m.group(1), []
            continue
        if not s or s[0] in ";." or s.endswith(":"):
            continue
        insts.append(s)
        if not ("buffer_load_dwordx4" in s and " lds" in s):
            continue
        ops = s.split(None, 1)[1].split(",")
        used = _sregs(",".join(ops[1:3])) | {"m0"}
        waits = 0
        for prev in reversed(insts[:-1]):
            if prev.startswith("s_nop"):
                waits += int(prev.split()[1], 0) + 1
            else:
                m2 = re.match(r"v_\w+\s+(s\[\d+:\d+\]|s\d+|m0)\b", prev)
                if m2 and _sregs(m2.group(1)) & used:
                    hits.append((func, i + 1, prev))
                    break
                waits += 1
            if waits >= 5:
                break
    return hits


def _check_hazards(src: str) -> None:
    with tempfile.TemporaryDirectory() as td:
        out = os.path.join(td, "k.s")
        cmd = [HIPCC, *DEVICE_FLAGS, "--cuda-device-only", "-S", src, "-o", out]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc -S failed for {src}:\n{r.stderr}")
        hits = lds_dma_hazards(open(out).read())
    if hits:
        lines = "\n".join(f"  {f}: line {ln}: {w}" for f, ln, w in hits[:10])
        raise RuntimeError(f"{src}: {len(hits)} LDS-DMA copies read an SGPR a VALU instruction "
                           f"wrote fewer than five wait states before (an s_nop 4 in front of "
                           f"those copies clears it):\n{lines}")


def build(verbose: bool = True) -> str:
    os.makedirs(os.path.join(LIBDIR, "obj"), exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = [os.path.join(LIBDIR, "obj", os.path.basename(s) + ".o") for s in srcs]
    dma_srcs = [s for s in srcs if "lds\"" in open(s).read() or "dma16" in open(s).read()]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs) + len(dma_srcs))) as ex:
        futs = [ex.submit(_compile, s, o) for s, o in zip(srcs, objs)]
        futs += [ex.submit(_check_hazards, s) for s in dma_srcs]
        for f in futs:
            f.result()
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
