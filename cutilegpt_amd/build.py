"""Build recipe for libcgpt.so (hand-written gfx950 HIP kernels + C ABI).

Compiles every ``csrc/*.hip`` with ``hipcc --offload-arch=gfx950`` into one
shared object next to this file.  Runs on a machine without a GPU (hipcc
cross-compiles).  ``python -m cutilegpt_amd.build`` or ``build()``.
"""

from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libcgpt.so")
BENCH_LIB = os.path.join(HERE, "libcgpt_bench.so")
ROOT = os.path.dirname(HERE)

ARCH = "gfx950"
# Packed fp32 VALU ops are kept out of the generated code (-packed-fp32-ops).
HIPCC_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the cutilegpt_amd kernels need ROCm's hipcc")


# Per-file flags.  Attention rescales and exponentiates its MFMA accumulators
# in the VALU every KV block; the VGPR form of the MFMAs keeps them out of the
# AGPRs (no v_accvgpr_read/write shuttling).
FILE_FLAGS = {
    "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: str, obj: str, extra) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), *extra,
           "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{res.stderr}")
    # hipcc's host pass does not know the packed-fp32 feature; drop that noise.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msg = "\n".join(l for l in res.stderr.splitlines() if noise not in l and l.strip())
    if msg:
        sys.stderr.write(msg + "\n")


def build(verbose: bool = False, extra_flags=()) -> str:
    """Compile all kernels and link ``libcgpt.so``; returns its path."""
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, os.path.basename(s)[:-4] + ".o") for s in srcs]
    workers = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        list(ex.map(lambda p: _compile(p[0], p[1], list(extra_flags)), zip(srcs, objs)))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of libcgpt.so failed:\n{res.stderr}")
    # Resolve every symbol now (a kernel whose host stub was not emitted shows
    # up as an undefined symbol only at dlopen time).
    chk = subprocess.run([sys.executable, "-c", f"import ctypes; ctypes.CDLL({tmp!r}, mode=2)"],
                         capture_output=True, text=True)
    if chk.returncode != 0:
        raise RuntimeError(f"libcgpt.so does not load:\n{chk.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_bench(extra_flags)
    return LIB


def build_bench(extra_flags=()) -> str:
    """``libcgpt_bench.so``: bench.py's bandwidth-ceiling probe (csrc_bench/),
    kept out of libcgpt.so's ABI."""
    src = os.path.join(HERE, "csrc_bench", "ceiling.hip")
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    obj = os.path.join(objdir, "bench_ceiling.o")
    _compile(src, obj, list(extra_flags))
    tmp = BENCH_LIB + ".tmp"
    res = subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, obj],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of libcgpt_bench.so failed:\n{res.stderr}")
    os.replace(tmp, BENCH_LIB)
    return BENCH_LIB


if __name__ == "__main__":
    build(verbose=True)
