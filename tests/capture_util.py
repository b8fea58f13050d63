"""Writes a capture directory in the reference's recorder format (tools/twin/stk_twin/rec.py:1-9, _ref at
rec.py:22-28), for the replay tests: ops.jsonl, one record a line, and blobs/<sha256> of raw contiguous bytes."""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

_NAMES = {np.dtype(np.uint16): "bfloat16", np.dtype(np.float32): "float32", np.dtype(np.int64): "int64",
          np.dtype(np.bool_): "bool"}


def ref(root: Path, a: np.ndarray, dtype: str | None = None) -> dict:
    data = np.ascontiguousarray(a).tobytes()
    sha = hashlib.sha256(data).hexdigest()
    (root / "blobs").mkdir(parents=True, exist_ok=True)
    p = root / "blobs" / sha
    if not p.exists():
        p.write_bytes(data)
    return {"sha": sha, "dtype": dtype or _NAMES[a.dtype], "shape": list(a.shape)}


def write(root: Path, records: list[dict]) -> None:
    """records: {name, kind, attrs, ins: {k: array}, outs: {k: array}} or {note: ...}; arrays as numpy (bf16 bits as
    uint16)."""
    root.mkdir(parents=True, exist_ok=True)
    lines = []
    for i, r in enumerate(records):
        if "note" in r:
            lines.append(json.dumps({"i": i, **r}))
            continue
        lines.append(json.dumps({"i": i, "name": r["name"], "kind": r["kind"], "attrs": r.get("attrs", {}),
                                 "ins": {k: ref(root, v) for k, v in r.get("ins", {}).items()},
                                 "outs": {k: ref(root, v) for k, v in r.get("outs", {}).items()}, "launches": []}))
    (root / "ops.jsonl").write_text("\n".join(lines) + "\n")
