"""Build libflexatt.so (the HIP kernels + C ABI) in-tree for gfx950.

Each kernel source is compiled once per head dim (-DFLEXATT_D=...) so the
template instances compile in parallel; the objects are linked into
``libflexatt.so`` next to this file.  Usage: ``python build_lib.py [-j N]``.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libflexatt.so")
HEAD_DIMS = (32, 64, 128, 256)
PER_D_SOURCES = ("fwd_mfma.hip", "fwd_ws.hip", "fwd_decode.hip", "bwd_mfma.hip", "bwd_kv.hip", "bwd_q.hip", "bwd_dq_ds.hip",
                  "f32_mfma.hip")
SINGLE_SOURCES = ("delta.hip", "capi.hip")
# Sources whose kernels load into registers through asm that the compiler
# does not know is in flight (load16_async): a VGPR spill could store or
# reuse such a register before its load lands, so their kernels must build
# without scratch.
NO_SCRATCH_SOURCES = ("bwd_dq_ds.hip",)


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def common_flags() -> list:
    return [
        "--offload-arch=gfx950",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # packed fp32 VALU forms are kept out of every kernel
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
    ]


def jobs() -> list:
    out = []
    for src in PER_D_SOURCES:
        for d in HEAD_DIMS:
            obj = os.path.join(OUT_DIR, f"{src[:-4]}_d{d}.o")
            out.append((os.path.join(CSRC, src), obj, [f"-DFLEXATT_D={d}"]))
    for src in SINGLE_SOURCES:
        out.append((os.path.join(CSRC, src), os.path.join(OUT_DIR, f"{src[:-4]}.o"), []))
    return out


def scratch_kernels(remarks: str) -> list:
    """(kernel, bytes per lane) for every kernel with scratch in -Rpass-analysis=kernel-resource-usage output."""
    out, name = [], None
    for line in remarks.splitlines():
        if "Function Name:" in line:
            name = line.split("Function Name:")[1].split()[0]
        elif "ScratchSize [bytes/lane]:" in line:
            n = int(line.split("ScratchSize [bytes/lane]:")[1].split()[0])
            if n > 0:
                out.append((name, n))
    return out


def _compile(job):
    src, obj, extra = job
    guard = os.path.basename(src) in NO_SCRATCH_SOURCES
    cmd = [hipcc()] + common_flags() + extra + (["-Rpass-analysis=kernel-resource-usage"] if guard else []) + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    if guard:
        bad = scratch_kernels(r.stderr)
        if bad:
            os.remove(obj)
            raise RuntimeError(f"{os.path.basename(src)} {' '.join(extra)}: kernels with asm register loads use scratch "
                               f"(a spilled register could be reused while its load is in flight): {bad}")
    return obj


def build(njobs: int | None = None, verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    njobs = njobs or min(16, os.cpu_count() or 4)
    todo = jobs()
    with ThreadPoolExecutor(max_workers=njobs) as ex:
        objs = list(ex.map(_compile, todo))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(objs)} objects")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    args = ap.parse_args()
    build(args.j, verbose=True)
    sys.exit(0)
