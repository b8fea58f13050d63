"""Build the gfx950 HIP library (liblr_attn.so) in-tree with hipcc.

The library is the product: the kernels under csrc/ and the C ABI of include/lr_attn.h. It is compiled for gfx950
only (MI355X / MI350X), with packed-fp32 instruction selection switched off.

    python -m localrouter_amd.build          # builds localrouter_amd/liblr_attn.so
"""
from __future__ import annotations

import concurrent.futures
import json
import os
import re
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

# Scratch (spill) budget per kernel, bytes per lane. The streaming attention kernel and the INT8 attention kernel count
# their direct global->LDS refills with explicit `s_waitcnt vmcnt(N)`; a scratch access among those loads would be
# counted too, and the waits would no longer name the loads they wait for. The streaming kernel keeps one 4-byte value
# in scratch (over key rows, attn_stream_kernel<true>, three), stored and reloaded only outside its streaming loop; the
# INT8 kernel at 128-key tiles three, around the peeled step of its last tile (the partial tile's P mask), the others
# none: the build generates their assembly and fails when a scratch access sits in a loop block (LOOP_SCAN,
# loop_scratch_ops). Every other kernel uses none. The build fails when a kernel needs more: the spill must then be
# found and removed, not accepted. The first entry whose name is part of the kernel's mangled name applies.
SCRATCH_BUDGET = {"attn_stream_kernelILb1E": 16, "attn_stream_kernel": 8, "i8_attn_kernel": 16}
REMARK_FLAGS = ["-Rpass-analysis=kernel-resource-usage"]
RESOURCES = PKG / "_build" / "resources.json"

# host-only C++ (the RoPE table builders of include/lr_rope.h): the system compiler, no contraction of f64 products
# and sums into FMAs, so that tables are the same bits as the numpy builders
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-ffp-contract=off"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build localrouter_amd)")


def kernel_resources(text: str) -> dict[str, dict[str, int]]:
    """The compiler's kernel-resource-usage remarks: {mangled kernel name: {"VGPRs": n, "AGPRs": n, "ScratchSize": n,
    ...}} (ScratchSize in bytes per lane)."""
    out: dict[str, dict[str, int]] = {}
    cur = None
    for line in text.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([A-Za-z ]+?)(?: \[bytes/lane\])?(?: \[waves/SIMD\])?: (\d+) \[-Rpass-analysis", line)
        if m and cur is not None:
            cur[m.group(1).strip()] = int(m.group(2))
    return out


def scratch_violations(res: dict[str, dict[str, int]]) -> list[str]:
    """Kernels whose scratch exceeds SCRATCH_BUDGET (0 for a kernel not listed)."""
    bad = []
    for name, r in res.items():
        budget = next((b for k, b in SCRATCH_BUDGET.items() if k in name), 0)
        if r.get("ScratchSize", 0) > budget:
            bad.append(f"{name}: {r.get('ScratchSize')} bytes of scratch per lane (budget {budget})")
    return bad


def loop_scratch_ops(asm: str, kernel: str) -> tuple[int, list[str]]:
    """(scratch instructions of `kernel`, those inside one of its loops) in the gfx950 assembly `asm`. A basic block is
    in a loop when the compiler's own block comment says so ("in Loop:" or "Loop Header"); a spill there would sit
    among the streaming loop's direct-to-LDS refills and be counted by their explicit vmcnt waits."""
    m = re.search(r"^(\S*" + re.escape(kernel) + r"\S*):", asm, re.M)
    if not m:
        raise RuntimeError(f"kernel {kernel} not found in the assembly")
    body = asm[m.start():asm.find(".Lfunc_end", m.start())].splitlines()
    total, inside, in_loop = 0, [], False
    for line in body:
        if re.match(r"^(\.LBB\S*:|; %bb\.\d+:)", line):
            in_loop = "in Loop:" in line or "Loop Header" in line
        if re.match(r"^\s+scratch_(load|store)", line):
            total += 1
            if in_loop:
                inside.append(line.strip())
    return total, inside


# kernels with a scratch budget: (source, kernel) whose assembly is scanned for scratch inside loops
LOOP_SCAN = [("attn_stream.hip", "attn_stream_kernel"), ("int8_attn.hip", "i8_attn_kernel")]


def _run(cmd: list[str]) -> str:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = [l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l]
    shown, in_remark = [], False   # the resource remarks and their source excerpts are parsed, not shown
    for l in lines:
        if "-Rpass-analysis=kernel-resource-usage" in l:
            in_remark = True
        elif not (in_remark and re.match(r"^\s*\d*\s*\|", l)):
            in_remark = False
            shown.append(l)
    out = "\n".join(shown)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return "\n".join(lines)


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
            cmd = [cc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), *REMARK_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), file=sys.stderr)
        cmds.append(cmd)
        objs.append(str(obj))
    # the sources compile independently: a few at a time (each hipcc process is single-threaded)
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", "0") or 0) or (os.cpu_count() or 1)))
    res: dict[str, dict[str, int]] = {}
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for f in [pool.submit(_run, c) for c in cmds]:
            res.update(kernel_resources(f.result()))
    RESOURCES.write_text(json.dumps(res, indent=1, sort_keys=True))
    bad = scratch_violations(res)
    if bad:
        raise RuntimeError("kernels over their scratch budget:\n  " + "\n  ".join(bad))
    # the kernels allowed a spill keep it outside their loops: their device assembly is generated and scanned
    for src, kernel in LOOP_SCAN:
        asm_path = objdir / (Path(src).stem + ".s")
        _run([cc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "--cuda-device-only", "-S", str(CSRC / src),
              "-o", str(asm_path)])
        asm = asm_path.read_text()
        for name in sorted(set(re.findall(r"^(_Z\S*" + re.escape(kernel) + r"\S*):", asm, re.M))):
            _, inside = loop_scratch_ops(asm, name)
            if inside:
                raise RuntimeError(f"{name}: scratch accesses inside a loop:\n  " + "\n  ".join(inside))
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, *LIBS, "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
