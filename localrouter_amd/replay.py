"""Replay gate for recorded twin captures: the attention-path ops of a capture run through this library.

The capture format is the reference's (tools/twin/stk_twin/rec.py:1-9): a directory with
  ops.jsonl   one op a line: {i, name, kind, attrs, ins: {k: ref}, outs: {k: ref}, launches: [...]}
              (non-op lines carry "note" instead of "kind")
  blobs/<sha> raw contiguous tensor bytes; a ref is {sha, dtype, shape} (rec.py:22-28)
The reference's gate (src/engines/qwen_image/replay.zig:1-3) replays every op of a capture through the Zig forward
and compares outputs byte for byte with its own CUDA kernels. This gate replays the ops on this library's path, each
from its captured inputs ("alone" mode) or, with --chained, from the outputs of the ops replayed before it whose
recorded outputs it consumed (matched by blob hash), and compares with the captured outputs to the attention bar (max-abs 2e-2,
mean-abs 2e-3 on bf16 outputs) -- other kernels than the twin's cannot be expected to round identically -- and also
reports how many outputs are byte-equal. Replayed kinds (tools/twin/stk_twin/dit.py:225-282):
  attention  q [B, N, H, D], k / v [B, S, HK, D] -> y [B, N, H * D]; attrs causal, and p0 / nkeys for a segment;
             scale 1 / sqrt(D). A masked SDPA record (attrs "masked", input "mask" boolean or additive, broadcast
             over [B, *, N, S]) is replayed when the mask is a key-padding mask (every query row the same: through
             lr_attention_kmask_bf16) or exactly causal; other masks are skipped.
  rms_rope   qkv [B, N, 3, H, D], w [D], cos / sin [N, D / 2] f32, attrs part (0 q, 1 k) and eps -> y [B, N, H, D]:
             per-head RMSNorm then interleaved-pair rotation (the Qwen engine's _rms_rope_kernel).
Every other kind is counted as skipped.

    python -m localrouter_amd.replay CAPTURE_DIR [--limit N] [--chained]
"""
from __future__ import annotations

import argparse
import json
import math
import sys
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

# rec.py writes str(t.dtype) without the "torch." prefix; bf16 is kept as its uint16 bit pattern here
_DTYPES = {"bfloat16": np.uint16, "float32": np.float32, "float16": np.float16, "int64": np.int64, "int32": np.int32,
           "uint8": np.uint8, "bool": np.bool_, "int8": np.int8}

BAR_MAX_ABS = 2e-2
BAR_MEAN_ABS = 2e-3


@dataclass
class Op:
    i: int
    name: str
    kind: str
    attrs: dict
    ins: dict
    outs: dict


@dataclass
class Stats:
    equal: int = 0
    within: int = 0
    differ: int = 0
    skipped: int = 0
    notes: list = field(default_factory=list)


def read_ops(root: str | Path) -> list[Op]:
    """The op records of a capture (notes dropped), in file order."""
    ops = []
    for line in (Path(root) / "ops.jsonl").read_text().splitlines():
        if not line.strip():
            continue
        r = json.loads(line)
        if "kind" not in r:
            continue
        ops.append(Op(r["i"], r["name"], r["kind"], r.get("attrs", {}), r.get("ins", {}), r.get("outs", {})))
    return ops


def load_ref(root: str | Path, ref: dict) -> np.ndarray:
    """A ref {sha, dtype, shape} as a numpy array (bf16 as uint16 bits)."""
    dt = _DTYPES.get(ref["dtype"])
    if dt is None:
        raise ValueError(f"unsupported dtype {ref['dtype']}")
    shape = tuple(ref["shape"])
    n = math.prod(shape)
    data = (Path(root) / "blobs" / ref["sha"]).read_bytes() if n else b""
    a = np.frombuffer(data, dtype=dt)
    if a.size != n:
        raise ValueError(f"blob {ref['sha'][:12]}: {a.size} elements, shape {shape} needs {n}")
    return a.reshape(shape)


def _bool(x) -> bool:
    return x in (True, 1, "1", "true", "True")


def compare(got_bits: np.ndarray, want_bits: np.ndarray) -> tuple[bool, bool, float, float]:
    """(byte-equal, within the bar, max-abs, mean-abs) of two bf16 bit arrays."""
    g = (got_bits.astype(np.uint32) << 16).view(np.float32)
    w = (want_bits.astype(np.uint32) << 16).view(np.float32)
    if g.shape != w.shape:
        return False, False, math.inf, math.inf
    d = np.abs(g.astype(np.float64) - w.astype(np.float64))
    mx, mean = (float(d.max()), float(d.mean())) if d.size else (0.0, 0.0)
    return bool(np.array_equal(got_bits, want_bits)), mx <= BAR_MAX_ABS and mean <= BAR_MEAN_ABS, mx, mean


def classify_mask(m: np.ndarray, B: int, N: int, S: int):
    """An SDPA mask (boolean, True keeps; or additive, 0 keeps) broadcast over [B, 1, N, S]: ("keys", keep [B, S])
    when every query row of a batch is the same (key padding), ("causal", None) when it is exactly lower-triangular
    over N == S, else (None, None) (per-head or other masks). A bf16 additive mask arrives as its uint16 bits (as
    load_ref returns it): +0.0 and -0.0 (0x8000, what (1 - keep) * -10000 gives for kept keys) both keep. A batch
    that keeps no key (SDPA gives NaN rows there) is not replayed: (None, None)."""
    if m.dtype == np.bool_:
        pass
    elif m.dtype == np.uint16:
        m = (m & 0x7FFF) == 0
    else:
        m = m.astype(np.float32) == 0.0
    if m.ndim > 4:
        return None, None
    try:
        m = np.broadcast_to(m, (B, 1, N, S))[:, 0]
    except ValueError:
        return None, None
    if (m == m[:, :1, :]).all():
        keep = np.ascontiguousarray(m[:, 0, :])
        if not keep.any(axis=1).all():
            return None, None
        return "keys", keep
    if N == S and (m == np.tril(np.ones((N, S), bool))[None]).all():
        return "causal", None
    return None, None


def replay_op(root: str | Path, op: Op, produced: dict | None = None):
    """Run one op through the library from its captured inputs; returns the output bits, or None if not replayed.
    produced: sha -> array; an input whose recorded blob is the recorded output of an op replayed earlier is taken
    from that op's replayed output instead (chained mode)."""
    import torch

    from . import ops

    def dev(name):
        ref = op.ins[name]
        a = produced[ref["sha"]] if produced and ref["sha"] in produced else load_ref(root, ref)
        a = a.reshape(tuple(ref["shape"]))
        t = torch.from_numpy(np.array(a))   # a writable copy of the read-only blob view
        return (t.view(torch.bfloat16) if a.dtype == np.uint16 else t).cuda()

    if op.kind == "attention":
        q, k, v = dev("q"), dev("k"), dev("v")
        B, N, H, D = q.shape
        S, HK = k.shape[1], k.shape[2]
        if D != ops.D:
            return None
        causal = _bool(op.attrs.get("causal", False))
        p0 = int(op.attrs.get("p0", 0))
        nkeys = int(op.attrs.get("nkeys", S))
        keep = None
        if "mask" in op.ins:
            how, keep = classify_mask(load_ref(root, op.ins["mask"]), B, N, S)
            if how is None:
                return None
            causal = causal or how == "causal"
        elif _bool(op.attrs.get("masked", False)):
            return None
        ys = []
        for b in range(B):
            if keep is not None:
                km = torch.from_numpy(keep[b].astype(np.uint8)).cuda()
                ys.append(ops.attention_kmask(q[b], k[b], v[b], km, n_valid=int(keep[b].sum()),
                                              scale=1.0 / math.sqrt(D)))
            else:
                ys.append(ops.attention(q[b], k[b], v[b], nkeys=nkeys, causal=causal, p0=p0, heads=H, kv_heads=HK,
                                        scale=1.0 / math.sqrt(D)))
        torch.cuda.synchronize()
        return torch.stack(ys).reshape(B, N, H * D).view(torch.int16).cpu().numpy().view(np.uint16)
    if op.kind == "rms_rope":
        qkv = dev("qkv")
        B, N, three, H, D = qkv.shape
        if three != 3 or D != ops.D:
            return None
        w = dev("w")
        if w.dtype == torch.bfloat16:
            w = w.float()
        cos, sin = dev("cos").float().contiguous(), dev("sin").float().contiguous()
        part = int(op.attrs.get("part", 0))
        eps = float(op.attrs.get("eps", 1e-6))
        dst = torch.empty((B, N, H, D), dtype=torch.bfloat16, device=qkv.device)
        ops.rms_rope(qkv, dst, w.contiguous(), n=N, heads=H, b=B, src_row_stride=3 * H * D, src_off=part * H * D,
                     dst_row_stride=H * D, src_b_stride=N * 3 * H * D, dst_b_stride=N * H * D,
                     table_kind=ops.TABLE_COSSIN_F32, table_a=cos, table_b=sin, table_row_stride=cos.stride(0),
                     rot=2 * cos.shape[1], pairing=ops.PAIR_INTERLEAVED, eps=eps)
        torch.cuda.synchronize()
        return dst.view(torch.int16).cpu().numpy().view(np.uint16)
    return None


def replay(root: str | Path, limit: int | None = None, log=print, chained: bool = False) -> Stats:
    """Alone: every op from its captured inputs. Chained: inputs that are outputs of ops replayed earlier come from
    those replayed outputs, so differences accumulate along the chain as they would in an engine."""
    st = Stats()
    produced = {} if chained else None
    for op in read_ops(root)[:limit]:
        got = replay_op(root, op, produced)
        if got is None:
            st.skipped += 1
            continue
        want = load_ref(root, op.outs["y"])
        if chained:
            produced[op.outs["y"]["sha"]] = got
        eq, ok, mx, mean = compare(got, want.reshape(got.shape) if want.size == got.size else want)
        if eq:
            st.equal += 1
        elif ok:
            st.within += 1
        else:
            st.differ += 1
        line = f"{op.i} {op.name} ({op.kind}): {'equal' if eq else 'within bar' if ok else 'DIFFERS'}" \
               f" max-abs {mx:.3g} mean-abs {mean:.3g}"
        st.notes.append(line)
        log(line)
    return st


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("capture")
    ap.add_argument("--limit", type=int, default=None)
    ap.add_argument("--chained", action="store_true", help="inputs from earlier replayed outputs")
    a = ap.parse_args(argv)
    st = replay(a.capture, a.limit, chained=a.chained)
    print(f"equal {st.equal}, within bar {st.within}, differ {st.differ}, skipped {st.skipped}")
    return 1 if st.differ else 0


if __name__ == "__main__":
    sys.exit(main())
