"""The engines' Zig side of the boundary, checked on the host (zig is not in this image, so the files are compared
with the C headers and the in-tree build instead of compiled):

  src/engines/hip/lr_attn.zig  every function of include/lr_attn.h, lr_rope.h and lr_mmdit.h declared extern with the
                               same name, the same number of arguments and matching argument kinds (pointers and
                               integers of the same width), and the same return kind;
  build/hip.zig                compiles exactly the sources localrouter_amd/build.py compiles, with the same flags.
"""
from __future__ import annotations

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
ZIG = ROOT / "src" / "engines" / "hip" / "lr_attn.zig"
BUILD = ROOT / "build" / "hip.zig"
HEADERS = [ROOT / "include" / h for h in ("lr_attn.h", "lr_rope.h", "lr_mmdit.h")]

# C type -> kind; pointers (and the stream handle) are 64-bit addresses on both sides
C_KIND = {"int": "i32", "float": "f32", "double": "f64", "int64_t": "i64", "size_t": "usize", "void": "void"}
ZIG_KIND = {"c_int": "i32", "f32": "f32", "f64": "f64", "i64": "i64", "usize": "usize", "void": "void", "u64": "ptr",
            "Stream": "ptr"}


def c_decls():
    out = {}
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b(int|size_t|int64_t|double|void)\s+(lr_\w+)\s*\(([^)]*)\)\s*;", text):
            args = [a.strip() for a in m.group(3).split(",")] if m.group(3).strip() not in ("", "void") else []
            kinds = ["ptr" if "*" in a or a.startswith("lr_stream_t") else C_KIND[a.rsplit(" ", 1)[0].replace("const ", "")]
                     for a in args]
            out[m.group(2)] = (C_KIND[m.group(1)], kinds)
    return out


def zig_decls():
    text = ZIG.read_text()
    out = {}
    for m in re.finditer(r'pub extern "lr_attn" fn (lr_\w+)\((.*?)\)\s*([\w\s\*\[\]]+?);', text, flags=re.S):
        args = [a.strip() for a in m.group(2).replace("\n", " ").split(",") if a.strip()]
        kinds = []
        for a in args:
            t = a.split(":", 1)[1].strip()
            kinds.append(ZIG_KIND.get(t, "ptr" if t.startswith(("*", "?", "[")) else t))
        out[m.group(1)] = (ZIG_KIND[m.group(3).strip()], kinds)
    return out


def test_every_c_function_has_its_zig_extern():
    c, z = c_decls(), zig_decls()
    assert len(c) >= 40
    assert sorted(c) == sorted(z), f"missing in zig: {sorted(set(c) - set(z))}, extra: {sorted(set(z) - set(c))}"
    for name, (ret, kinds) in c.items():
        zret, zkinds = z[name]
        assert zret == ret, f"{name}: returns {zret} in zig, {ret} in C"
        assert zkinds == kinds, f"{name}: arguments {zkinds} in zig, {kinds} in C"


def test_zig_constants_match_the_headers():
    text = ZIG.read_text()
    attn = (ROOT / "include" / "lr_attn.h").read_text()
    for name in ("TABLE_NONE", "TABLE_COSSIN_F32", "TABLE_MAT2_BF16", "TABLE_MAT2_F32", "PAIR_INTERLEAVED",
                 "PAIR_SPLIT_HALF", "WEIGHT_NONE", "WEIGHT_F32", "WEIGHT_BF16"):
        c_val = re.search(rf"#define LR_{name} (\d+)", attn).group(1)
        z_val = re.search(rf"pub const {name}: c_int = (\d+);", text).group(1)
        assert c_val == z_val, name
    for c_name, z_name in (("LR_ATTN_CFG_AUTO", "CFG_AUTO"), ("LR_ATTN_CFG_PIPE_W8", "CFG_PIPE_W8"),
                           ("LR_ATTN_CFG_PIPE_W4", "CFG_PIPE_W4"), ("LR_ATTN_CFG_STREAM_W8", "CFG_STREAM_W8"),
                           ("LR_ATTN_ABI_VERSION", "ABI_VERSION")):
        assert re.search(rf"#define {c_name} (\d+)", attn).group(1) == \
            re.search(rf"pub const {z_name}: c_int = (\d+);", text).group(1), c_name
    split = re.search(r"#define LR_JOINT_SPLIT_BYTES \(\(size_t\)(\d+)\)", attn).group(1)
    assert re.search(r"pub const JOINT_SPLIT_BYTES: usize = (\d+);", text).group(1) == split


def test_mmdit_weights_struct_matches():
    """lr_mmdit_weights / lr_mmdit_stream_weights field order (extern structs are passed by pointer)."""
    h = (ROOT / "include" / "lr_mmdit.h").read_text()
    z = ZIG.read_text()
    for c_struct, z_struct in (("lr_mmdit_stream_weights", "MmditStream"), ("lr_mmdit_weights", "MmditWeights")):
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (c_struct, c_struct), h, flags=re.S).group(1)
        c_fields = re.findall(r"(?:\*|\s)(\w+)(?:,\s*(\w+))?;", re.sub(r"/\*.*?\*/", "", body, flags=re.S))
        c_names = [n for pair in c_fields for n in pair if n]
        z_body = re.search(r"pub const %s = extern struct \{(.*?)\};" % z_struct, z).group(1)
        z_names = re.findall(r"(\w+):", z_body)
        assert c_names == z_names, (c_struct, c_names, z_names)


def test_build_hip_zig_matches_the_in_tree_build():
    from localrouter_amd import build
    text = BUILD.read_text()
    zig_sources = re.findall(r'\.file = "([\w.]+)"', text)
    hip_sources = [s for s in build.SOURCES if s.endswith(".hip")]
    assert sorted(zig_sources) == sorted(hip_sources)
    assert 'kernels/hip/rope_host.cpp' in text and "-ffp-contract=off" in text and "-lhipblaslt" in text
    for flag in build.HIPCC_FLAGS:
        assert f'"{flag}"' in text, flag
    for src, extra in build.EXTRA_FLAGS.items():
        line = next(l for l in text.splitlines() if f'.file = "{src}"' in l)
        assert all(f'"{f}"' in line for f in extra), src


def test_engine_tree_layout_matches_build_hip_zig(tmp_path):
    """localrouter_amd.engine_tree lays the sources out as the kernels/hip tree build/hip.zig compiles: every file
    build/hip.zig names exists there, the Zig module and headers sit where it and the sources expect them, and every
    source of the tree preprocesses (its includes, ../../include/lr_*.h among them, resolve inside the tree)."""
    import shutil
    import subprocess

    from localrouter_amd import engine_tree
    written = engine_tree.lay_out(tmp_path)
    assert written
    text = BUILD.read_text()
    named = set(re.findall(r'\.file = "([\w.]+)"', text)) | set(re.findall(r'kernels/hip/([\w.]+)"', text))
    assert "attn_stream.hip" in named and "rope_host.cpp" in named
    for f in named:
        assert (tmp_path / "kernels" / "hip" / f).is_file(), f
    assert (tmp_path / "build" / "hip.zig").read_text() == text
    assert re.search(r'b\.path\("src/engines/hip/lr_attn\.zig"\)', text)
    assert (tmp_path / "src" / "engines" / "hip" / "lr_attn.zig").is_file()
    for h in HEADERS:
        assert (tmp_path / "include" / h.name).read_bytes() == h.read_bytes()
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        return
    for f in sorted(named):
        src = tmp_path / "kernels" / "hip" / f
        cmd = ([hipcc, "-std=c++17", "-E", "--cuda-host-only"] if f.endswith(".hip") else
               [shutil.which("g++") or "g++", "-std=c++17", "-E"])
        r = subprocess.run(cmd + [str(src), "-o", "/dev/null"], capture_output=True, text=True)
        assert r.returncode == 0, f"{f}: {r.stderr[-2000:]}"
