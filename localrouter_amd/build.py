"""Build the gfx950 HIP library (liblr_attn.so) in-tree with hipcc.

The library is the product: the kernels under csrc/ and the C ABI of include/lr_attn.h. It is compiled for gfx950
only (MI355X / MI350X), with packed-fp32 instruction selection switched off.

    python -m localrouter_amd.build          # builds localrouter_amd/liblr_attn.so
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "liblr_attn.so"
SOURCES = ["attn_fwd.hip", "attn_stream.hip", "kv_image.hip", "rms_rope.hip", "int8_attn.hip", "keys.hip", "lr_abi.hip",
           "mmdit.hip", "rope_host.cpp"]
# libraries the shared object links: hipBLASLt for the MMDiT block's projections and MLP
LIBS = ["-L/opt/rocm/lib", "-lhipblaslt"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 (v_pk_*_f32) selection off for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# per-source extra flags: the streaming kernel's fully unrolled key-tile step is larger than clang's default limit for
# `#pragma unroll`, and a partly unrolled step would index its register arrays at run time
EXTRA_FLAGS = {"attn_stream.hip": ["-mllvm", "-pragma-unroll-threshold=1000000"]}

# host-only C++ (the RoPE table builders of include/lr_rope.h): the system compiler, no contraction of f64 products
# and sums into FMAs, so that tables are the same bits as the numpy builders
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-ffp-contract=off"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build localrouter_amd)")


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source to an object, then link liblr_attn.so. Always recompiles."""
    cc = hipcc()
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    objs, cmds = [], []
    for src in SOURCES:
        obj = objdir / (Path(src).stem + ".o")
        if src.endswith(".cpp"):
            cmd = [shutil.which("g++") or "g++", *CXX_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
        else:
            cmd = [cc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), file=sys.stderr)
        cmds.append(cmd)
        objs.append(str(obj))
    # the sources compile independently: a few at a time (each hipcc process is single-threaded)
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", "0") or 0) or (os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for f in [pool.submit(_run, c) for c in cmds]:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, *LIBS, "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
