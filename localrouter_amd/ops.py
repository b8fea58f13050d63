"""torch-facing host interface, mirroring the reference engine's kernel bindings.

  attention(...)        <- Ops.attention, src/engines/qwen_image/ops_launch.zig:163-172
  rms_rope(...)         <- Triton.ropeRun + Rope, src/engines/qwen_image/triton_k.zig:44-53
  rms_rope_qk(...)      <- Kitchen.rmsRope, src/engines/minimax_h3/launch.zig:421-441
  joint_attention(...)  <- Dit.block's rope_q / rope_k / V copy / attention chain, src/engines/qwen_image/dit.zig:252-293
  joint_kv_prepare(...), joint_attention_prepared(...)  <- its two stages (keys / values reused across calls)
  joint_q_prepare(...), joint_attention_images(...)     <- the fused op's query and attention launches one by one
  joint_prepare(...)                                    <- its first launch (queries, keys and values) as one call
  int8_attention(...)   <- MiniMax H3's INT8 attention, kitchen_int8_attention{,_rows}
                           (kernels/cuda/minimax/kitchen_launch.cu:193-280)
  kitchen_attention(...), kitchen_attention_prep(...), kitchen_attention_kernel(...)
                        <- Kitchen.attention / attentionPrep / attentionKernel on a packed qkv buffer,
                           src/engines/minimax_h3/launch.zig:351-419

Every call validates shapes on the host, then goes through the C ABI (liblr_attn.so) on torch's current HIP stream.
torch supplies device memory and the stream handle only; all compute is the library's HIP kernels.
"""
from __future__ import annotations

import math

import torch

from . import _lib

D = 128
TABLE_NONE, TABLE_COSSIN_F32, TABLE_MAT2_BF16, TABLE_MAT2_F32 = 0, 1, 2, 3
PAIR_INTERLEAVED, PAIR_SPLIT_HALF = 0, 1
WEIGHT_NONE, WEIGHT_F32, WEIGHT_BF16 = 0, 1, 2
CFG_AUTO, CFG_PIPE_W8, CFG_PIPE_W4, CFG_STREAM_W8 = 0, 1, 2, 9
SCALE_128 = float(torch.tensor(1.0 / math.sqrt(128.0), dtype=torch.float32))  # f32 1/sqrt(128) = 0x3DB504F3


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _rows(t: torch.Tensor, name: str, heads: int | None = None) -> int:
    """A bf16 CUDA tensor viewed as rows [n, heads, 128] with unit stride inside a row; returns its row stride."""
    if not t.is_cuda or t.dtype != torch.bfloat16:
        raise ValueError(f"{name}: expected a bf16 tensor on the GPU, got {t.dtype} on {t.device}")
    if t.dim() == 3:
        n, h, d = t.shape
        if d != D or t.stride(2) != 1 or (h > 1 and t.stride(1) != D):
            raise ValueError(f"{name}: expected [n, heads, 128] with contiguous heads, got {tuple(t.shape)} / {t.stride()}")
        if heads is not None and h != heads:
            raise ValueError(f"{name}: {h} heads, expected {heads}")
        return t.stride(0)
    if t.dim() == 2:
        if t.stride(1) != 1:
            raise ValueError(f"{name}: rows must be contiguous")
        return t.stride(0)
    raise ValueError(f"{name}: expected a 2-D or 3-D tensor")


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor | None = None, *, w: int | None = None,
              heads: int | None = None, kv_heads: int | None = None, nkeys: int | None = None, causal: bool = False,
              p0: int = 0, scale: float = SCALE_128, config: int = CFG_AUTO) -> torch.Tensor:
    """q [w, heads, 128], k / v [>= nkeys, kv_heads, 128] -> out [w, heads, 128] (bf16 rows; query head h reads kv
    head h / (heads / kv_heads)); causal: query i (position p0 + i) sees keys 0..p0 + i, else all nkeys keys."""
    w = q.shape[0] if w is None else w
    heads = q.shape[1] if heads is None else heads
    kv_heads = k.shape[1] if kv_heads is None else kv_heads
    nkeys = k.shape[0] if nkeys is None else nkeys
    q_rs = _rows(q, "q", heads)
    k_rs = _rows(k, "k", kv_heads)
    v_rs = _rows(v, "v", kv_heads)
    if out is None:
        out = torch.empty((w, heads, D), dtype=torch.bfloat16, device=q.device)
    o_rs = _rows(out, "out", heads)
    if k.shape[0] < nkeys or v.shape[0] < nkeys or q.shape[0] < w or out.shape[0] < w:
        raise ValueError("attention: tensors shorter than w / nkeys")
    _lib.call("lr_attention_bf16_ex", _ptr(q), _ptr(k), _ptr(v), _ptr(out), p0, w, heads, kv_heads, nkeys,
              int(causal), scale, q_rs, k_rs, v_rs, o_rs, D, D, config, _stream())
    return out


def attention_ws_bytes(w: int, heads: int, nkeys: int, causal: bool = False) -> int:
    """lr_attention_ws_bytes: the workspace lr_attention_bf16_ws uses (0: none)."""
    return int(_lib.load().lr_attention_ws_bytes(w, heads, nkeys, int(causal)))


def attention_ws(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor | None = None, *,
                 causal: bool = False, p0: int = 0, scale: float = SCALE_128,
                 workspace: torch.Tensor | None = None) -> torch.Tensor:
    """lr_attention_bf16_ws: attention over key and value rows with device scratch: non-causal calls of at most 32
    query blocks split over the keys (flash-decoding), others of at least 4,096 keys run the streaming kernel over the
    key rows with its split tail, the rest run as lr_attention_bf16; q [w, heads, 128], k / v [nkeys, kv_heads, 128]
    with the same row stride. A workspace of attention_ws_bytes is allocated when none is given."""
    w, heads = q.shape[0], q.shape[1]
    nkeys, kv_heads = k.shape[0], k.shape[1]
    q_rs, k_rs = _rows(q, "q", heads), _rows(k, "k", kv_heads)
    if _rows(v, "v", kv_heads) != k_rs:
        raise ValueError("attention_ws: k and v need the same row stride")
    if out is None:
        out = torch.empty((w, heads, D), dtype=torch.bfloat16, device=q.device)
    o_rs = _rows(out, "out", heads)
    nb = attention_ws_bytes(w, heads, nkeys, causal)
    if workspace is None and nb:
        workspace = torch.empty(nb, dtype=torch.uint8, device=q.device)
    _lib.call("lr_attention_bf16_ws", _ptr(q), _ptr(k), _ptr(v), _ptr(out), p0, w, heads, kv_heads, nkeys,
              int(causal), scale, q_rs, k_rs, o_rs, _ptr(workspace), 0 if workspace is None else workspace.numel(),
              _stream())
    return out


def attention_kmask(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kmask: torch.Tensor | None,
                    out: torch.Tensor | None = None, *, n_valid: int | None = None, scale: float = SCALE_128,
                    workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Kandinsky-6's attention with a key-padding mask: q [w, heads, 128], k / v [nkeys, kv_heads, 128] (the same row
    stride), kmask u8 [nkeys] on the GPU (nonzero = keep) or None; n_valid = the number of kept keys (computed here,
    with a device sync, when not given; the engine knows it on the host)."""
    w, heads = q.shape[0], q.shape[1]
    nkeys, kv_heads = k.shape[0], k.shape[1]
    q_rs = _rows(q, "q", heads)
    k_rs = _rows(k, "k", kv_heads)
    if _rows(v, "v", kv_heads) != k_rs:
        raise ValueError("attention_kmask: k and v need the same row stride")
    if out is None:
        out = torch.empty((w, heads, D), dtype=torch.bfloat16, device=q.device)
    o_rs = _rows(out, "out", heads)
    ws_ptr, ws_bytes = None, 0
    if kmask is not None:
        if kmask.dtype != torch.uint8 or not kmask.is_cuda or kmask.numel() < nkeys:
            raise ValueError("kmask: expected u8 [nkeys] on the GPU")
        if n_valid is None:
            n_valid = int((kmask[:nkeys] != 0).sum().item())
        ws_bytes = int(_lib.load().lr_attention_kmask_workspace_bytes(n_valid, kv_heads))
        if workspace is None:
            workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        ws_ptr = _ptr(workspace)
        ws_bytes = workspace.numel()
    else:
        n_valid = nkeys
    _lib.call("lr_attention_kmask_bf16", _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(kmask), n_valid, w, heads,
              kv_heads, nkeys, scale, q_rs, k_rs, o_rs, ws_ptr, ws_bytes, _stream())
    return out


def rms_rope(src: torch.Tensor, dst: torch.Tensor, w: torch.Tensor | None, *, n: int, heads: int, b: int = 1,
             src_row_stride: int, src_off: int = 0, dst_row_stride: int, src_b_stride: int = 0,
             dst_b_stride: int = 0, table_kind: int = TABLE_COSSIN_F32, table_a: torch.Tensor | None = None,
             table_b: torch.Tensor | None = None, table_row_stride: int | None = None, rot: int = 128,
             pairing: int = PAIR_INTERLEAVED, eps: float = 1e-6, round_norm: bool = False) -> torch.Tensor:
    """Triton.ropeRun's contract with element strides: dst[bi, r, h] = rope(rmsnorm(src[bi*sb + r*srs + off + h*128]))."""
    for t, nm in ((src, "src"), (dst, "dst")):
        if not t.is_cuda or t.dtype != torch.bfloat16:
            raise ValueError(f"{nm}: expected bf16 on the GPU")
    w_kind = WEIGHT_NONE if w is None else (WEIGHT_F32 if w.dtype == torch.float32 else WEIGHT_BF16)
    if w is not None and (w.numel() < D or not w.is_contiguous()):
        raise ValueError("w: expected a contiguous [128] tensor")
    if table_row_stride is None:
        table_row_stride = 0 if table_a is None else table_a.stride(0)
    _lib.call("lr_rms_rope_bf16", _ptr(src), src_row_stride, src_off, _ptr(dst), dst_row_stride, n, b, src_b_stride,
              dst_b_stride, heads, _ptr(w), w_kind, table_kind, _ptr(table_a), _ptr(table_b), table_row_stride, rot,
              pairing, eps, int(round_norm), _stream())
    return dst


def rms_rope_qk(q: torch.Tensor, k: torch.Tensor, q_norm: torch.Tensor, k_norm: torch.Tensor, freqs: torch.Tensor, *,
                heads: int, seq: int, rot: int = 96, eps: float = 1e-5) -> None:
    """Kitchen.rmsRope: q, k [seq, heads, 128] views (packed qkv allowed) normalised and rotated in place with bf16
    weights and a bf16 [seq, rot/2, 2, 2] table (split-half pairs)."""
    q_rs = _rows(q, "q", heads)
    k_rs = _rows(k, "k", heads)
    if freqs.dtype != torch.bfloat16 or q_norm.dtype != torch.bfloat16 or k_norm.dtype != torch.bfloat16:
        raise ValueError("rms_rope_qk: bf16 weights and table expected")
    f_rs = freqs.stride(0)
    _lib.call("lr_rms_rope_qk_bf16", _ptr(q), _ptr(k), seq, heads, q_rs, k_rs, _ptr(q_norm), _ptr(k_norm),
              _ptr(freqs), f_rs, rot, eps, _stream())


def workspace_bytes(sk: int, kv_heads: int) -> int:
    """lr_joint_attention_workspace_bytes: key and value tile images, 2 * HK * ceil(Sk / 64) * 16 KB."""
    return int(_lib.load().lr_joint_attention_workspace_bytes(sk, kv_heads))


def joint_attention(q_raw: torch.Tensor, k_raw: torch.Tensor, v: torch.Tensor, out: torch.Tensor | None = None, *,
                    q_norm: torch.Tensor | None = None, k_norm: torch.Tensor | None = None,
                    table_kind: int = TABLE_COSSIN_F32, q_table: tuple | None = None, k_table: tuple | None = None,
                    pairing: int = PAIR_INTERLEAVED, rot: int = 128, eps: float = 1e-6, causal: bool = False,
                    p0: int = 0, scale: float = SCALE_128, n_pre: int = 0, workspace: torch.Tensor | None = None,
                    config: int = CFG_AUTO) -> torch.Tensor:
    """The fused op: per-head QK-RMSNorm + RoPE + attention. q_raw [Sq, H, 128], k_raw / v [Sk, HK, 128] bf16 rows;
    q_table / k_table = (table_a, table_b) (table_b None for the 2x2 kinds; k_table defaults to q_table)."""
    Sq, H = q_raw.shape[0], q_raw.shape[1]
    Sk, HK = k_raw.shape[0], k_raw.shape[1]
    q_rs, k_rs, v_rs = _rows(q_raw, "q_raw", H), _rows(k_raw, "k_raw", HK), _rows(v, "v", HK)
    if v.shape[0] < Sk:
        raise ValueError("v shorter than k")
    if out is None:
        out = torch.empty((Sq, H, D), dtype=torch.bfloat16, device=q_raw.device)
    o_rs = _rows(out, "out", H)
    for t, nm in ((q_norm, "q_norm"), (k_norm, "k_norm")):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != D):
            raise ValueError(f"{nm}: expected fp32 [128]")
    qa = qb = ka = kb = None
    stride = 0
    if table_kind != TABLE_NONE:
        if q_table is None:
            raise ValueError("joint_attention: q_table required")
        k_table = q_table if k_table is None else k_table
        qa, qb = q_table
        ka, kb = k_table
        stride = qa.stride(0)
        if ka.stride(0) != stride:
            raise ValueError("q and k tables must share a row stride")
    need = workspace_bytes(Sk, HK)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q_raw.device)
    if workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace: {need} bytes needed")
    _lib.call("lr_joint_attention_fused_ex", _ptr(q_raw), _ptr(k_raw), _ptr(v), _ptr(out), _ptr(q_norm),
              _ptr(k_norm), table_kind, _ptr(qa), _ptr(qb), _ptr(ka), _ptr(kb), stride, pairing, rot, eps, Sq, Sk, H,
              HK, p0, int(causal), scale, q_rs, k_rs, v_rs, o_rs, n_pre, _ptr(workspace),
              workspace.numel() * workspace.element_size(), config, _stream())
    return out


def joint_kv_prepare(k_raw: torch.Tensor, v: torch.Tensor, workspace: torch.Tensor, *,
                     k_norm: torch.Tensor | None = None, table_kind: int = TABLE_COSSIN_F32,
                     k_table: tuple | None = None, pairing: int = PAIR_INTERLEAVED, rot: int = 128, eps: float = 1e-6,
                     n_pre: int = 0) -> torch.Tensor:
    """First stage of joint_attention: k_raw [Sk, HK, 128] normalised and rotated (rows < n_pre copied) and v laid out
    as tile images in the workspace (lr_joint_kv_prepare). Returns the workspace."""
    Sk, HK = k_raw.shape[0], k_raw.shape[1]
    k_rs, v_rs = _rows(k_raw, "k_raw", HK), _rows(v, "v", HK)
    if v.shape[0] < Sk:
        raise ValueError("v shorter than k")
    if k_norm is not None and (k_norm.dtype != torch.float32 or not k_norm.is_contiguous() or k_norm.numel() != D):
        raise ValueError("k_norm: expected fp32 [128]")
    ka = kb = None
    stride = 0
    if table_kind != TABLE_NONE:
        if k_table is None:
            raise ValueError("joint_kv_prepare: k_table required")
        ka, kb = k_table
        stride = ka.stride(0)
    nbytes = workspace.numel() * workspace.element_size()
    if nbytes < workspace_bytes(Sk, HK):
        raise ValueError(f"workspace: {workspace_bytes(Sk, HK)} bytes needed")
    _lib.call("lr_joint_kv_prepare", _ptr(k_raw), k_rs, _ptr(v), v_rs, _ptr(k_norm), table_kind, _ptr(ka), _ptr(kb),
              stride, pairing, rot, eps, Sk, HK, n_pre, _ptr(workspace), nbytes, _stream())
    return workspace


def joint_attention_prepared(q_raw: torch.Tensor, workspace: torch.Tensor, sk: int, kv_heads: int,
                             out: torch.Tensor | None = None, *, q_norm: torch.Tensor | None = None,
                             table_kind: int = TABLE_COSSIN_F32, q_table: tuple | None = None,
                             pairing: int = PAIR_INTERLEAVED, rot: int = 128, eps: float = 1e-6, causal: bool = False,
                             p0: int = 0, scale: float = SCALE_128, config: int = CFG_AUTO) -> torch.Tensor:
    """Second stage of joint_attention: q_raw [Sq, H, 128] over a workspace filled by joint_kv_prepare
    (lr_joint_attention_prepared)."""
    Sq, H = q_raw.shape[0], q_raw.shape[1]
    q_rs = _rows(q_raw, "q_raw", H)
    if out is None:
        out = torch.empty((Sq, H, D), dtype=torch.bfloat16, device=q_raw.device)
    o_rs = _rows(out, "out", H)
    if q_norm is not None and (q_norm.dtype != torch.float32 or not q_norm.is_contiguous() or q_norm.numel() != D):
        raise ValueError("q_norm: expected fp32 [128]")
    qa = qb = None
    stride = 0
    if table_kind != TABLE_NONE:
        if q_table is None:
            raise ValueError("joint_attention_prepared: q_table required")
        qa, qb = q_table
        stride = qa.stride(0)
    _lib.call("lr_joint_attention_prepared", _ptr(q_raw), _ptr(workspace), workspace.numel() * workspace.element_size(),
              _ptr(out), _ptr(q_norm), table_kind, _ptr(qa), _ptr(qb), stride, pairing, rot, eps, Sq, sk, H, kv_heads,
              p0, int(causal), scale, q_rs, o_rs, config, _stream())
    return out


def joint_q_prepare(q_raw: torch.Tensor, q_prep: torch.Tensor | None = None, *, q_norm: torch.Tensor | None = None,
                    table_kind: int = TABLE_COSSIN_F32, q_table: tuple | None = None,
                    pairing: int = PAIR_INTERLEAVED, rot: int = 128, eps: float = 1e-6) -> torch.Tensor:
    """The fused op's query launch (lr_joint_q_prepare): q_raw [Sq, H, 128] normalised and rotated, rounded once to
    bf16, into q_prep (q_raw itself is allowed: in place)."""
    Sq, H = q_raw.shape[0], q_raw.shape[1]
    q_rs = _rows(q_raw, "q_raw", H)
    if q_prep is None:
        q_prep = torch.empty((Sq, H, D), dtype=torch.bfloat16, device=q_raw.device)
    p_rs = _rows(q_prep, "q_prep", H)
    if q_norm is not None and (q_norm.dtype != torch.float32 or not q_norm.is_contiguous() or q_norm.numel() != D):
        raise ValueError("q_norm: expected fp32 [128]")
    qa = qb = None
    stride = 0
    if table_kind != TABLE_NONE:
        if q_table is None:
            raise ValueError("joint_q_prepare: q_table required")
        qa, qb = q_table
        stride = qa.stride(0)
    _lib.call("lr_joint_q_prepare", _ptr(q_raw), q_rs, _ptr(q_prep), p_rs, _ptr(q_norm), table_kind, _ptr(qa),
              _ptr(qb), stride, pairing, rot, eps, Sq, H, _stream())
    return q_prep


def joint_prepare(q_raw: torch.Tensor, k_raw: torch.Tensor, v: torch.Tensor, workspace: torch.Tensor,
                  q_prep: torch.Tensor | None = None, *, q_norm: torch.Tensor | None = None,
                  k_norm: torch.Tensor | None = None, table_kind: int = TABLE_COSSIN_F32, q_table: tuple | None = None,
                  k_table: tuple | None = None, pairing: int = PAIR_INTERLEAVED, rot: int = 128, eps: float = 1e-6,
                  n_pre: int = 0) -> torch.Tensor:
    """The fused op's first launch (lr_joint_prepare): joint_q_prepare and joint_kv_prepare as one launch. Returns
    q_prep (allocated when None)."""
    Sq, H = q_raw.shape[0], q_raw.shape[1]
    Sk, HK = k_raw.shape[0], k_raw.shape[1]
    q_rs, k_rs, v_rs = _rows(q_raw, "q_raw", H), _rows(k_raw, "k_raw", HK), _rows(v, "v", HK)
    if q_prep is None:
        q_prep = torch.empty((Sq, H, D), dtype=torch.bfloat16, device=q_raw.device)
    p_rs = _rows(q_prep, "q_prep", H)
    for name, w in (("q_norm", q_norm), ("k_norm", k_norm)):
        if w is not None and (w.dtype != torch.float32 or not w.is_contiguous() or w.numel() != D):
            raise ValueError(f"{name}: expected fp32 [128]")
    qa = qb = ka = kb = None
    stride = 0
    if table_kind != TABLE_NONE:
        if q_table is None or k_table is None:
            raise ValueError("joint_prepare: q_table and k_table required")
        (qa, qb), (ka, kb) = q_table, k_table
        if qa.stride(0) != ka.stride(0):
            raise ValueError("q and k tables must share a row stride")
        stride = qa.stride(0)
    nbytes = workspace.numel() * workspace.element_size()
    _lib.call("lr_joint_prepare", _ptr(q_raw), q_rs, _ptr(q_prep), p_rs, _ptr(k_raw), k_rs, _ptr(v), v_rs,
              _ptr(q_norm), _ptr(k_norm), table_kind, _ptr(qa), _ptr(qb), _ptr(ka), _ptr(kb), stride, pairing, rot, eps,
              Sq, Sk, H, HK, n_pre, _ptr(workspace), nbytes, _stream())
    return q_prep


def joint_attention_images(q_prep: torch.Tensor, workspace: torch.Tensor, sk: int, kv_heads: int,
                           out: torch.Tensor | None = None, *, causal: bool = False, p0: int = 0,
                           scale: float = SCALE_128) -> torch.Tensor:
    """The fused op's attention launch (lr_joint_attention_images): queries prepared by joint_q_prepare over a
    workspace filled by joint_kv_prepare. out may be q_prep itself."""
    Sq, H = q_prep.shape[0], q_prep.shape[1]
    p_rs = _rows(q_prep, "q_prep", H)
    if out is None:
        out = torch.empty((Sq, H, D), dtype=torch.bfloat16, device=q_prep.device)
    o_rs = _rows(out, "out", H)
    _lib.call("lr_joint_attention_images", _ptr(q_prep), p_rs, _ptr(workspace),
              workspace.numel() * workspace.element_size(), _ptr(out), o_rs, Sq, sk, H, kv_heads, p0, int(causal),
              scale, _stream())
    return out


# ------------------------------------------------------------------------------------------------ INT8 chain
def int8_scale(head_dim: int) -> float:
    """head_dim^-0.5 rounded to fp32, the scale the reference's callers pass (0x3DB504F3 for 128)."""
    return float(torch.tensor(1.0 / math.sqrt(head_dim), dtype=torch.float32))


def int8_workspace_bytes(heads: int, sq: int, *, sk: int | None = None, kv_heads: int | None = None,
                         batch: int = 1, head_dim: int = D) -> int:
    """Kitchen.Plan.of(heads, S).total for this library's workspace layout (0 when the case is unsupported)."""
    sk = sq if sk is None else sk
    kv_heads = heads if kv_heads is None else kv_heads
    return int(_lib.load().lr_int8_attention_workspace_bytes(batch, heads, kv_heads, sq, sk, head_dim))


def _bhsd(t: torch.Tensor, name: str) -> tuple[int, int, int]:
    if not t.is_cuda or t.dtype != torch.bfloat16:
        raise ValueError(f"{name}: expected a bf16 tensor on the GPU, got {t.dtype} on {t.device}")
    if t.dim() != 4 or t.shape[3] not in (64, 128) or t.stride(3) != 1:
        raise ValueError(f"{name}: expected [B, heads, S, 64 or 128] with unit last stride, got {tuple(t.shape)} / "
                         f"{t.stride()}")
    return t.stride(0), t.stride(1), t.stride(2)


def _workspace(workspace: torch.Tensor | None, need: int, device) -> torch.Tensor:
    if need == 0:
        raise ValueError("int8 attention: unsupported sizes")
    if workspace is None:
        return torch.empty(need, dtype=torch.uint8, device=device)
    if workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"int8 attention: workspace of {workspace.numel() * workspace.element_size()} bytes, need {need}")
    return workspace


def int8_attention_prep(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        workspace: torch.Tensor | None = None) -> torch.Tensor:
    """The K anchor, Q / K rotation and int8 quantisation, V per-channel int8 into the workspace (returned)."""
    B, H, Sq, d = q.shape
    HK, Sk = k.shape[1], k.shape[2]
    qs, ks, vs = _bhsd(q, "q"), _bhsd(k, "k"), _bhsd(v, "v")
    workspace = _workspace(workspace, int8_workspace_bytes(H, Sq, sk=Sk, kv_heads=HK, batch=B, head_dim=d), q.device)
    _lib.call("lr_int8_attention_prep", _ptr(q), _ptr(k), _ptr(v), _ptr(workspace), B, H, HK, Sq, Sk, d, *qs, *ks,
              *vs, _stream())
    return workspace


def int8_attention_prep_rope(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_norm: torch.Tensor,
                             k_norm: torch.Tensor, freqs: torch.Tensor, *, rot: int = 96, eps: float = 1e-6,
                             workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Kitchen.rmsRope fused into the prep (lr_int8_attention_prep_rope): the workspace int8_attention_prep would
    write after rms_rope_qk(q, k, ...) in place, with q and k left unmodified. q_norm / k_norm bf16 [128], freqs bf16
    [S, >= 2 * rot] ([rot/2][2][2] per row); head dim 128, Sq == Sk."""
    B, H, Sq, d = q.shape
    HK, Sk = k.shape[1], k.shape[2]
    qs, ks, vs = _bhsd(q, "q"), _bhsd(k, "k"), _bhsd(v, "v")
    for t, nm in ((q_norm, "q_norm"), (k_norm, "k_norm"), (freqs, "freqs")):
        if not t.is_cuda or t.dtype != torch.bfloat16 or t.stride(-1) != 1:
            raise ValueError(f"{nm}: expected bf16 on the GPU with unit last stride")
    workspace = _workspace(workspace, int8_workspace_bytes(H, Sq, sk=Sk, kv_heads=HK, batch=B, head_dim=d), q.device)
    _lib.call("lr_int8_attention_prep_rope", _ptr(q), _ptr(k), _ptr(v), _ptr(workspace), B, H, HK, Sq, Sk, d, *qs,
              *ks, *vs, _ptr(q_norm), _ptr(k_norm), _ptr(freqs), freqs.stride(0), rot, eps, _stream())
    return workspace


def kitchen_attention_prep_rope(qkv: torch.Tensor, workspace: torch.Tensor | None, heads: int, freqs: torch.Tensor,
                                q_norm: torch.Tensor, k_norm: torch.Tensor, rot: int = 96,
                                eps: float = 1e-6) -> torch.Tensor:
    """Kitchen.rmsRope + Kitchen.attentionPrep on one packed qkv buffer, as one prep (qkv is not modified)."""
    q, k, v = qkv_views(qkv, heads)
    return int8_attention_prep_rope(q, k, v, q_norm, k_norm, freqs, rot=rot, eps=eps, workspace=workspace)


def int8_attention_kernel(workspace: torch.Tensor, out: torch.Tensor, *, batch: int, heads: int, kv_heads: int,
                          sq: int, sk: int, scale: float | None = None, rows: bool = False,
                          head_dim: int = D) -> torch.Tensor:
    """The attention over a workspace int8_attention_prep filled; out [B, H, Sq, d] or rows [Sq, H * d] (B 1); the
    scale defaults to d^-0.5 in fp32."""
    if not out.is_cuda or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("out: expected a contiguous bf16 tensor on the GPU")
    scale = int8_scale(head_dim) if scale is None else scale
    _lib.call("lr_int8_attention_kernel", _ptr(out), _ptr(workspace), batch, heads, kv_heads, sq, sk, head_dim, scale,
              1 if rows else 0, _stream())
    return out


def int8_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor | None = None, *,
                   scale: float | None = None, rows: bool = False,
                   workspace: torch.Tensor | None = None) -> torch.Tensor:
    """kitchen_int8_attention: q [B, H, Sq, d], k / v [B, HK, Sk, d] bf16 views (any strides, unit last; d 64 or
    128) -> out [B, H, Sq, d] bf16, or rows [Sq, H * d] when rows (B 1); the scale defaults to d^-0.5 in fp32."""
    B, H, Sq, d = q.shape
    HK, Sk = k.shape[1], k.shape[2]
    qs, ks, vs = _bhsd(q, "q"), _bhsd(k, "k"), _bhsd(v, "v")
    scale = int8_scale(d) if scale is None else scale
    workspace = _workspace(workspace, int8_workspace_bytes(H, Sq, sk=Sk, kv_heads=HK, batch=B, head_dim=d), q.device)
    if out is None:
        out = torch.empty((Sq, H * d) if rows else (B, H, Sq, d), dtype=torch.bfloat16, device=q.device)
    name = "lr_int8_attention_rows" if rows else "lr_int8_attention"
    _lib.call(name, _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(workspace), B, H, HK, Sq, Sk, d, *qs, *ks, *vs, scale,
              _stream())
    return out


def qkv_views(qkv: torch.Tensor, heads: int, head_dim: int = D) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """q, k, v [1, heads, S, d] views of a packed qkv buffer [S, 3 * heads * d] (launch.zig:362-366)."""
    S = qkv.shape[0]
    parts = qkv.view(S, 3, heads, head_dim)
    return tuple(parts[:, i].permute(1, 0, 2).unsqueeze(0) for i in range(3))


def kitchen_attention_prep(qkv: torch.Tensor, workspace: torch.Tensor | None, heads: int,
                           head_dim: int = D) -> torch.Tensor:
    """Kitchen.attentionPrep(qkv, ws, heads, seq)."""
    return int8_attention_prep(*qkv_views(qkv, heads, head_dim), workspace)


def kitchen_attention_kernel(out: torch.Tensor, workspace: torch.Tensor, heads: int, seq: int,
                             rows: bool, head_dim: int = D) -> torch.Tensor:
    """Kitchen.attentionKernel(out, ws, heads, seq, rows)."""
    return int8_attention_kernel(workspace, out, batch=1, heads=heads, kv_heads=heads, sq=seq, sk=seq, rows=rows,
                                 head_dim=head_dim)


def kitchen_attention(qkv: torch.Tensor, heads: int, out: torch.Tensor | None = None,
                      workspace: torch.Tensor | None = None, rows: bool = False, head_dim: int = D) -> torch.Tensor:
    """Kitchen.attention(qkv, out, ws, heads, seq): out [heads, S, d] (rows: [S, heads * d])."""
    S = qkv.shape[0]
    o = int8_attention(*qkv_views(qkv, heads, head_dim), None if out is None else out.view(
        (S, heads * head_dim) if rows else (1, heads, S, head_dim)), rows=rows, workspace=workspace)
    return o if rows else o.view(heads, S, head_dim)
