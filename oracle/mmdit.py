"""CPU oracle of the MMDiT double-stream block forward (include/lr_mmdit.h) -- TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's cpu_baseline leg may import this module, and only as the checker.

The reference has no double-stream block (its Qwen engine is single-stream, src/engines/qwen_image/dit.zig:242-308),
so the block's composition is this build's own definition, restated here in numpy fp32 with the GPU path's bf16
rounding points (every step's output is rounded to bf16, as the library stores it). Its pieces follow the reference
where it has them:
  * sinusoid: kernels/cuda/qwen_image/ops.cu:84-99 (t * 1000 rounded to bf16, / 1000 by reciprocal multiply, rounded
    again, * 1000; freq_i = exp(-ln(1e4) i / 128); cos | sin);
  * GELU-tanh: ops.cu:48-57 (torch's operation order);
  * gated residual: ops.cu:25-31 (x = fma(a, g, x));
  * SiLU: ops.cu:34-39;
  * the joint attention with QK-RMSNorm and RoPE: the attention oracle of this package (liblro.so).
Pinning (tests/test_oracle_mmdit.py): the sinusoid and GELU against their closed forms and special values, the
LayerNorm against its moments, the linear layout against a brute-force loop, the adaLN-zero identity (zero
modulation weights leave both streams unchanged), and the meaning of each modulation chunk on zero inputs, where the
LayerNorm is 0: a scale has no effect, a shift does, and a zero gate shuts its own branch and only that one (planted
shift/scale and gate swaps fail these). The composition itself has no reference to be pinned to: parity unpinned
beyond those checks.
"""
from __future__ import annotations

import numpy as np

from . import PAIR_INTERLEAVED, TABLE_COSSIN_F32, bf16_to_f32, f32_to_bf16, joint_attention

LN_EPS = np.float32(1e-6)


def bf16r(x: np.ndarray) -> np.ndarray:
    """fp32 values rounded to bf16 (nearest even), returned as fp32."""
    return bf16_to_f32(f32_to_bf16(np.asarray(x, np.float32)))


def sinusoid(t: float) -> np.ndarray:
    """emb [256] fp32 (bf16 values) from timestep t (ops.cu:84-99)."""
    f = np.float32
    tr = bf16r(np.array([f(t) * f(1000.0)], np.float32))[0]
    tr = bf16r(np.array([tr * f(1.0 / 1000.0)], np.float32))[0]
    tr = f(tr * f(1000.0))
    j = np.arange(256)
    i = (j & 127).astype(np.float32)
    freq = np.exp((f(-9.210340371976184) * i) * f(1.0 / 128.0)).astype(np.float32)
    arg = (tr * freq).astype(np.float32)
    return bf16r(np.where(j < 128, np.cos(arg), np.sin(arg)).astype(np.float32))


def silu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float32)
    return bf16r(x / (np.float32(1.0) + np.exp(-x)))


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), torch's order (ops.cu:48-57), fp32."""
    x = np.asarray(x, np.float32)
    beta = np.float32(1.4142135623730951 * 1.1283791670955126 * 0.5)
    inner = beta * (np.float32(0.044715) * (x * x * x) + x)
    return ((np.float32(0.5) * x) * (np.float32(1.0) + np.tanh(inner))).astype(np.float32)


def linear(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """x [M, K] fp32, w [N, K] (torch nn.Linear layout) -> x w^T [M, N], fp32 accumulation, rounded to bf16."""
    return bf16r(np.asarray(x, np.float32) @ np.asarray(w, np.float32).T)


def layer_norm_modulate(x: np.ndarray, shift: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """LayerNorm (no affine, eps 1e-6, two-pass fp32 moments) * (1 + scale) + shift, rounded to bf16."""
    x = np.asarray(x, np.float32)
    mean = x.mean(axis=1, dtype=np.float64).astype(np.float32)[:, None]
    d = x - mean
    var = (d.astype(np.float64) ** 2).mean(axis=1).astype(np.float32)[:, None]
    rstd = np.float32(1.0) / np.sqrt(var + LN_EPS)
    return bf16r(d * rstd * (np.float32(1.0) + scale[None, :]) + shift[None, :])


def gated_residual(x: np.ndarray, a: np.ndarray, g: np.ndarray) -> np.ndarray:
    """fma(a, g, x) rounded to bf16 (ops.cu:25-31); the fused multiply-add is taken in f64, one rounding to f32."""
    return bf16r((a.astype(np.float64) * g[None, :].astype(np.float64) + x.astype(np.float64)).astype(np.float32))


# the six modulation chunks of a stream, in the order of its mod projection's rows (include/lr_mmdit.h)
MOD_CHUNKS = ("shift_attn", "scale_attn", "gate_attn", "shift_mlp", "scale_mlp", "gate_mlp")


def mmdit_block(txt: np.ndarray, img: np.ndarray, w: dict, t: float, cos: np.ndarray, sin: np.ndarray,
                precise_attention: bool = False, chunk_order=(0, 1, 2, 3, 4, 5)):
    """One block. txt [St, D], img [Si, D]: uint16 bf16 bits. w: bf16 bits (uint16) arrays t1 [D, 256], t2 [D, D],
    and per stream s in (txt, img): s.mod [6D, D], s.qkv [3D, D], s.out [D, D], s.mlp_up [F, D], s.mlp_down [D, F];
    q_norm, k_norm [128] fp32. cos, sin [St + Si, 64] fp32. Returns (txt, img) fp32 arrays of bf16 values.
    chunk_order[i] is the chunk of the mod projection that serves as MOD_CHUNKS[i]; anything but the identity is a
    planted mistake, for the tests that show the semantic checks catch one."""
    W = {k: (bf16_to_f32(v) if v.dtype == np.uint16 else np.asarray(v, np.float32)) for k, v in w.items()}
    xt, xi = bf16_to_f32(txt), bf16_to_f32(img)
    St, D = xt.shape
    Si = xi.shape[0]
    S, H = St + Si, D // 128

    emb = sinusoid(t)[None, :]
    temb = linear(silu(linear(emb, W["t1"])), W["t2"])
    ts = silu(temb)
    mod = {s: linear(ts, W[f"{s}.mod"])[0] for s in ("txt", "img")}

    def chunk(s, i):
        i = chunk_order[i]
        return mod[s][i * D:(i + 1) * D]

    xs = {"txt": xt, "img": xi}
    # attention half
    hn = {s: layer_norm_modulate(xs[s], chunk(s, 0), chunk(s, 1)) for s in xs}
    qkv = np.concatenate([linear(hn["txt"], W["txt.qkv"]), linear(hn["img"], W["img.qkv"])])   # [S, 3D]
    bits = f32_to_bf16(qkv).reshape(S, 3, H, 128)
    attn = joint_attention(bits[:, 0], bits[:, 1], bits[:, 2], wq=W["q_norm"], wk=W["k_norm"],
                           table_kind=TABLE_COSSIN_F32, qa=cos, qb=sin, pairing=PAIR_INTERLEAVED, rot=128, eps=1e-6,
                           precise=precise_attention)
    attn = bf16r(attn.reshape(S, D))
    rows = {"txt": slice(0, St), "img": slice(St, S)}
    for s in xs:
        o = linear(attn[rows[s]], W[f"{s}.out"])
        xs[s] = gated_residual(xs[s], o, chunk(s, 2))
    # MLP half
    for s in xs:
        h = layer_norm_modulate(xs[s], chunk(s, 3), chunk(s, 4))
        m = linear(bf16r(gelu_tanh(linear(h, W[f"{s}.mlp_up"]))), W[f"{s}.mlp_down"])
        xs[s] = gated_residual(xs[s], m, chunk(s, 5))
    return xs["txt"], xs["img"]


def block_flops(n_txt: int, n_img: int, hidden: int, mlp: int) -> float:
    """GEMM + attention FLOPs of one block (the elementwise work not counted): per row 2 D (3D + D + 2F), the
    modulation and time vectors, and 4 S^2 D for the joint attention."""
    S = n_txt + n_img
    gemm = 2.0 * S * hidden * (3 * hidden + hidden + 2 * mlp)
    vec = 2.0 * (256 * hidden + hidden * hidden + 2 * 6 * hidden * hidden)
    return gemm + vec + 4.0 * S * S * hidden
