"""Lay this repository's HIP path out as the engine tree that build/hip.zig compiles.

    python -m localrouter_amd.engine_tree DEST [--symlink]

DEST is a LocalRouter checkout (or any directory). build/hip.zig compiles `kernels/hip/<file>` for every device
source and `kernels/hip/rope_host.cpp`, and its sources include `../../include/lr_*.h`; the Zig module is
`src/engines/hip/lr_attn.zig`. This script writes exactly that layout:

    DEST/kernels/hip/         every file of localrouter_amd/csrc (the .hip sources, their .inc / .h parts, rope_host.cpp)
    DEST/include/             lr_attn.h, lr_mmdit.h, lr_rope.h
    DEST/build/hip.zig        the build module (the root build.zig calls hip.lrAttn(b, target, optimize))
    DEST/src/engines/hip/     lr_attn.zig (the extern declarations)

Files are copied (or symlinked with --symlink, so that the engine tree follows this repository). Existing files of
the same names are replaced; nothing else in DEST is touched. Returns / prints the list of files written.
"""
from __future__ import annotations

import argparse
import os
import shutil
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent

# (source directory, glob, destination directory relative to DEST)
LAYOUT = [
    (PKG / "csrc", "*", "kernels/hip"),
    (ROOT / "include", "lr_*.h", "include"),
    (ROOT / "build", "hip.zig", "build"),
    (ROOT / "src" / "engines" / "hip", "*.zig", "src/engines/hip"),
]


def lay_out(dest: Path, symlink: bool = False) -> list[Path]:
    dest = Path(dest)
    written = []
    for src_dir, pattern, rel in LAYOUT:
        out_dir = dest / rel
        out_dir.mkdir(parents=True, exist_ok=True)
        for src in sorted(src_dir.glob(pattern)):
            if not src.is_file():
                continue
            dst = out_dir / src.name
            if dst.is_symlink() or dst.exists():
                dst.unlink()
            if symlink:
                os.symlink(src, dst)
            else:
                shutil.copy2(src, dst)
            written.append(dst)
    return written


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("dest", type=Path)
    ap.add_argument("--symlink", action="store_true")
    args = ap.parse_args()
    for p in lay_out(args.dest, args.symlink):
        print(p)


if __name__ == "__main__":
    main()
