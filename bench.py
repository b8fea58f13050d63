"""Benchmark of the DiT joint-attention hot path on one MI355X (gfx950).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--preroll-s SECONDS]
                    [--workload qwen-step|plumbing|edit|video|qwen21|h3-int8|mmdit|k6|rows] [--no-cpu-baseline]

A step is one lr_joint_attention_fused call over one synthetic batch: the preparation launch (keys RMSNorm + RoPE into
the workspace's tile images, queries RMSNorm + RoPE into the output rows), then the persistent streaming attention
kernel over them and the value rows. After the W warm-up steps, fused calls run untimed for a fixed --preroll-s seconds
(1 s by default, whatever W is), so that the timed region starts at the GPU's working clock; the line states both. The
K timed steps are K such calls back to back, with HIP events only before and after them; `value` and `ms_per_step`
come from those. A second loop of K calls made through the stage entry points (lr_joint_prepare, which also copies the
value rows into the workspace so that it holds everything the attention reads, then lr_joint_attention_images), with
an event between the two launches, times the attention kernel alone for `roofline` and the preparation
(`staged_ms_per_step`, `kernels_ms`). Inputs are resident in HBM before timing.
The default workload is BASELINE's Qwen-Image-style step: B=1, 24 heads x 128, 512 text + 4096 image tokens (64x64
grid, 2D RoPE on image tokens, text un-rotated), non-causal, QK-RMSNorm eps 1e-6 with weights 1.0, scale f32(1/sqrt(128)).

Prints ONE JSON line on stdout (everything else goes to stderr). FLOPs per call = 4 * Sq * Sk * 128 * H (QK^T + PV;
softmax, RMSNorm and RoPE not counted). `roofline` is the attention kernel (attn_stream_kernel) alone, timed with HIP
events on the stream it is launched on, against MI355X's published dense bf16 peak of 2.5 PFLOP/s; its `traffic` and
the shader clock come from the committed rocprofv3 PMC summary of the same command (profiles/). `cpu_baseline` times
the CPU oracle's fp32 flash-style path (OpenMP, every core the process may use) on a bounded sample of query rows of
the same workload, as a reported baseline only.

--workload qwen21 is the reference's own call shape (Qwen-Image 2.1, dit.zig:252-293): 4,096 image queries, 32 heads,
over an 80-key cached text prefix (already rotated, used as given: n_pre = 80) plus the 4,096 image keys.

--workload h3-int8 measures MiniMax H3's INT8 attention instead (5,967 tokens x 56 heads, the reference's headline
shape for it): a step is H3's whole chain on one packed qkv buffer (dit.zig:665-671), Kitchen.rmsRope fused into the
prep (lr_int8_attention_prep_rope: norm, rotary, anchor, Hadamard rotation, int8 Q / K / V) then the attention kernel
(lr_int8_attention_kernel, rows output); the unfused chain (lr_rms_rope_qk_bf16, lr_int8_attention_prep, the kernel)
is timed beside it. Ops per call = 4 * S^2 * 128 * H; `roofline` is the attention kernel against MI355X's dense int8
peak of 5.0 POP/s; `cpu_baseline` is the CPU oracle of the same chain (rmsRope + prep + fp64 attention over the
quantised operands) on a sample of heads and rows.

--workload mmdit measures BASELINE configs[2], the MMDiT double-stream block forward at the same shape (512 text +
4096 image tokens, hidden 3072, 24 heads, GELU-tanh MLP 12288, adaLN-zero modulation from the 256-d time sinusoid,
weights N(0, 0.02), activations N(0, 1)): a step is one lr_mmdit_block_bf16 call (in place on the two streams).
FLOPs per block = the GEMMs + the joint attention (elementwise work not counted). `roofline` is the block's largest
GEMM (the image stream's MLP up-projection, 4096 x 12288 x 3072) timed alone through lr_mmdit_linear_bf16;
`cpu_baseline` is the numpy fp32 oracle of the whole block (multithreaded BLAS) on the same inputs.

--workload k6 measures Kandinsky-6's attention calls (src/engines/kandinsky6/dit/launch.zig:260-300): a step is one
call of each of the four unmasked shapes its flash dispatch takes (visual self-attention 50,220 x 32 heads,
video-from-audio 50,220 <- 218 keys x 32 heads, audio-from-video 218 <- 50,220 keys x 16 heads, audio self 218 x 16
heads; rows of heads x 128, scale f32(1/sqrt(128))), each through lr_attention_bf16_ws, the library's route for
attention over key and value rows with device scratch. FLOPs per step = the sum of 4 * Sq * Sk * 128 * H. `roofline`
is the visual self-attention (the streaming kernel over key rows, attn_stream_kernel<true>, 99 % of the FLOPs) timed
alone; `cpu_baseline` is the CPU oracle's fp32 flash path on a sample of the visual call's query rows.

--workload rows measures the drop-in for the engines' Ops.attention (ops_launch.zig:163-172, pattn2_kernel) at
BASELINE's shape: q, k, v as rows [4608, 24, 128] bf16 N(0, 1), no norm or rotary (the caller's), non-causal, scale
f32(1/sqrt(128)); a step is one lr_attention_bf16 call with the library's own kernel choice (AUTO). The tile
configurations it chooses between (LR_ATTN_CFG_PIPE_W8, _PIPE_W4, _STREAM_W8) and lr_attention_bf16_ws (the split
tail over the workspace) are timed beside it on the same inputs. `roofline` is the AUTO call's kernel;
`cpu_baseline` the CPU oracle's fp32 flash path on sampled query rows.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0
PEAK_INT8_TOPS = 5000.0
METRIC = "attention TFLOP/s + % bf16 MFMA peak; ms/call at 4096+512 tokens, 24x128"
# the attention kernel of the fused call, as rocprofv3 names it
KERNEL = "attn_stream_kernel"
WORKLOADS = {
    # name: (text tokens, grid description, heads)
    "plumbing": dict(n_text=256, kind="grid2d", gh=32, gw=32, heads=24),
    "qwen-step": dict(n_text=512, kind="grid2d", gh=64, gw=64, heads=24),
    "edit": dict(n_text=512, kind="edit", frames=3, gh=64, gw=64, heads=24),
    "video": dict(n_text=512, kind="video3d", t=49, gh=44, gw=80, heads=24),
    # the reference's own call shape (Qwen-Image 2.1, src/engines/qwen_image/dit.zig:252-293): 4096 image queries over
    # an 80-row cached text prefix (keys already rotated, copied as they are) plus the 4096 image keys, 32 heads
    "qwen21": dict(n_text=80, kind="prefix2d", gh=64, gw=64, heads=32),
}
# seconds of back-to-back fused calls run after --warmup and before the timed region, whatever --warmup is: the
# shader clock ramps up over the first ~100 ms of a busy GPU, and a timed region that starts on a cold GPU measures
# that ramp rather than the kernel (a 5-call warm-up gave 0.312 ms per call, 300 calls 0.2625 ms, same box and build)
PREROLL_S = 1.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def tables(w):
    """The workload's cos/sin tables, from the library's host RoPE builders (bit-equal to localrouter_amd.rope)."""
    from localrouter_amd import rope_host as rope
    if w["kind"] == "grid2d":
        return rope.grid2d_table(w["n_text"], w["gh"], w["gw"])
    if w["kind"] == "edit":
        return rope.edit_table(w["n_text"], w["frames"], w["gh"], w["gw"])
    if w["kind"] == "prefix2d":   # the image rows of a text + image table: queries and the keys behind the prefix
        cos, sin = rope.grid2d_table(w["n_text"], w["gh"], w["gw"])
        return cos[w["n_text"]:].copy(), sin[w["n_text"]:].copy()
    return rope.video3d_table(w["n_text"], w["t"], w["gh"], w["gw"])


def from_profile(name: str, kernel: str, field: str = "traffic_bytes_per_launch"):
    """A figure of the committed rocprofv3 PMC summary profiles/<kernel>_<name>_pmc.md (None if absent)."""
    p = ROOT / "profiles" / f"{kernel}_{name}_pmc.md"
    if not p.exists():
        return None
    m = re.search(field + r":\s*([0-9.eE+]+)", p.read_text())
    return float(m.group(1)) if m else None


def traffic_from_profile(name: str, kernel: str):
    return from_profile(name, kernel)


def host_cpus():
    """(threads the CPU baseline uses, CPUs this process may run on, CPU model). The thread count is the process's
    CPU share: OMP_NUM_THREADS when set (the GPU boxes set it to their share), else every CPU of the affinity mask."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(avail, int(env)) if env.isdigit() and int(env) > 0 else avail
    model = ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return threads, avail, model


def cpu_baseline(q_bits, k_bits, v_bits, cos, sin, Sq, H, flops_per_row, n_pre=0, budget_s=10.0):
    """The oracle's fp32 flash-style path (norm + rope + attention) on a sample of query rows, timed on host cores.
    Query row i uses table row i; key j >= n_pre uses table row j - n_pre, keys j < n_pre are used as given."""
    import numpy as np

    import oracle
    threads = host_cpus()[0]
    oracle.set_threads(threads)
    rng = np.random.default_rng(0)
    Sk = k_bits.shape[0]

    def run(rows):
        t0 = time.perf_counter()
        # the reference's chain: q and k normalised, rotated and stored as bf16, then the attention
        qh = oracle.rms_rope(q_bits[rows], None, table_kind=oracle.TABLE_COSSIN_F32, ta=cos[rows], tb=sin[rows])
        kh = oracle.rms_rope(k_bits[n_pre:], None, table_kind=oracle.TABLE_COSSIN_F32, ta=cos[:Sk - n_pre],
                             tb=sin[:Sk - n_pre])
        qh = oracle.bf16_to_f32(oracle.f32_to_bf16(qh))
        kh = oracle.bf16_to_f32(oracle.f32_to_bf16(kh))
        if n_pre:
            kh = np.concatenate([oracle.bf16_to_f32(k_bits[:n_pre]), kh])
        vf = oracle.bf16_to_f32(v_bits)
        # all Sk keys for each sampled query row: the sampled rows are renumbered 0..n-1 (non-causal, so equivalent)
        out = oracle.attention(qh, kh, vf, precise=False)
        return time.perf_counter() - t0, out

    probe = np.sort(rng.choice(Sq, size=64, replace=False))
    dt, _ = run(probe)
    rate = 64 * flops_per_row / dt
    # as many query rows as fit in a third of the budget (all of them for the image shapes), then repeated runs of that
    # sample until the budget is spent; the median run is reported
    n = int(min(Sq, max(64, budget_s / 3 * rate / flops_per_row)) // 32 * 32)
    rows = np.sort(rng.choice(Sq, size=n, replace=False))
    times, out, spent = [], None, 0.0
    while spent < budget_s or len(times) < 3:
        dt, out = run(rows)
        times.append(dt)
        spent += dt
    dt = float(np.median(times))
    return dict(value=n * flops_per_row / dt / 1e12, threads=threads, rows=rows, out=out, seconds=dt, runs=len(times))


def preroll(call, seconds: float):
    """Back-to-back calls for `seconds` of wall time, so that the timed region starts on a GPU already at its working
    clock (synchronised every batch of calls: about 50 ms of work, at least one call). Returns (calls made, seconds
    spent); seconds 0 makes no call."""
    import torch
    if seconds <= 0:
        return 0, 0.0
    t0, calls, batch = time.perf_counter(), 0, 1
    while True:
        t1 = time.perf_counter()
        for _ in range(batch):
            call()
        calls += batch
        torch.cuda.synchronize()
        now = time.perf_counter()
        if now - t0 >= seconds:
            return calls, now - t0
        per = (now - t1) / batch
        batch = max(1, min(200, int(0.05 / max(per, 1e-6))))


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="qwen-step",
                    choices=sorted(WORKLOADS) + ["h3-int8", "mmdit", "k6", "rows"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--operands", default="randn", choices=["randn", "zeros"],
                    help="q, k, v data: randn = N(0, 1) (BASELINE's, the default); zeros = all zero, a power study: the "
                         "same kernels and schedule with operands that toggle no multiplier bits (not a BASELINE "
                         "measurement)")
    ap.add_argument("--preroll-s", type=float, default=PREROLL_S,
                    help="seconds of untimed calls after the warm-up and before timing (the GPU's clock settles)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one 256 MiB device-to-device copy after timing (the known-size kernel that scales "
                         "rocprofv3's FETCH_SIZE / WRITE_SIZE into bytes)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); the "
              "joint attention shards by heads with no exchange, so N GPUs would run this same kernel at H/N heads.",
              file=sys.stderr)
        sys.exit(2)

    if args.operands != "randn" and args.workload in ("h3-int8", "mmdit", "k6", "rows"):
        raise SystemExit("bench.py: --operands applies to the joint-attention workloads")
    if args.workload == "h3-int8":
        return bench_int8(args)
    if args.workload == "mmdit":
        return bench_mmdit(args)
    if args.workload == "k6":
        return bench_k6(args)
    if args.workload == "rows":
        return bench_rows(args)

    import numpy as np
    import torch

    from localrouter_amd import _lib, ops

    w = WORKLOADS[args.workload]
    H = w["heads"]
    cos_np, sin_np = tables(w)
    # queries: the table's rows; keys: an n_pre-row cached prefix (already rotated: used as given) plus one key per
    # query row (key j >= n_pre uses table row j - n_pre)
    n_pre = w["n_text"] if w["kind"] == "prefix2d" else 0
    Sq = cos_np.shape[0]
    Sk = n_pre + Sq
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    L = _lib.load()
    rc = L.lr_attn_init()
    if rc != 0:
        raise SystemExit(f"lr_attn_init: {rc} (not a gfx950?)")
    props = torch.cuda.get_device_properties(dev)
    log(f"[bench] device {props.name} {getattr(props, 'gcnArchName', '')} CUs {props.multi_processor_count}; "
        f"workload {args.workload}: Sq={Sq} Sk={Sk} (prefix {n_pre}) H={H}")

    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    q = torch.randn((Sq, H, 128), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    k = torch.randn((Sk, H, 128), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn((Sk, H, 128), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    if args.operands == "zeros":
        q.zero_(), k.zero_(), v.zero_()
    out = torch.empty_like(q)
    cos = torch.from_numpy(cos_np).to(dev)
    sin = torch.from_numpy(sin_np).to(dev)
    wq = torch.ones(128, dtype=torch.float32, device=dev)
    wk = torch.ones(128, dtype=torch.float32, device=dev)
    ws_bytes = ops.workspace_bytes(Sk, H)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    eps, scale, rs = 1e-6, ops.SCALE_128, H * 128

    def prepare():
        _lib.call("lr_joint_prepare", q.data_ptr(), rs, out.data_ptr(), rs, k.data_ptr(), rs, v.data_ptr(), rs,
                  wq.data_ptr(), wk.data_ptr(), ops.TABLE_COSSIN_F32, cos.data_ptr(), sin.data_ptr(), cos.data_ptr(),
                  sin.data_ptr(), 64, ops.PAIR_INTERLEAVED, 128, eps, Sq, Sk, H, H, n_pre, ws.data_ptr(), ws_bytes, sh)

    def attn():
        _lib.call("lr_joint_attention_images", out.data_ptr(), rs, ws.data_ptr(), ws_bytes, out.data_ptr(), rs, Sq, Sk,
                  H, H, 0, 0, scale, sh)

    def fused():
        _lib.call("lr_joint_attention_fused", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), wq.data_ptr(),
                  wk.data_ptr(), ops.TABLE_COSSIN_F32, cos.data_ptr(), sin.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                  64, ops.PAIR_INTERLEAVED, 128, eps, Sq, Sk, H, H, 0, 0, scale, rs, rs, rs, rs, n_pre, ws.data_ptr(),
                  ws_bytes, sh)

    for _ in range(args.warmup):
        fused()
        prepare()
        attn()
    torch.cuda.synchronize()
    pre_calls, pre_s = preroll(fused, args.preroll_s)
    log(f"[bench] warmup {args.warmup} done, pre-roll {pre_calls} calls in {pre_s:.2f} s; timing {args.steps} steps")

    K = args.steps
    # the timed steps: K fused calls, events around the whole loop only
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    e0.record(stream)
    for _ in range(K):
        fused()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms_step = e0.elapsed_time(e1) / K
    # the same K calls as their two launches with an event between them: the attention kernel and the preparation
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * K + 1)]
    torch.cuda.synchronize()
    for i in range(K):
        ev[2 * i].record(stream)
        prepare()
        ev[2 * i + 1].record(stream)
        attn()
    ev[2 * K].record(stream)
    torch.cuda.synchronize()
    t_prep = [ev[2 * i].elapsed_time(ev[2 * i + 1]) for i in range(K)]
    t_attn = [ev[2 * i + 1].elapsed_time(ev[2 * i + 2]) for i in range(K)]
    staged_ms = ev[0].elapsed_time(ev[2 * K]) / K
    flops = 4.0 * Sq * Sk * 128 * H
    attn_ms = float(np.mean(t_attn))
    prep_ms = float(np.mean(t_prep))
    value = flops / (ms_step * 1e-3) / 1e12
    achieved = flops / (attn_ms * 1e-3) / 1e12
    # the committed profiles are of N(0,1) operands; on zeros the clock is higher (the operand power study)
    clock = from_profile(args.workload, KERNEL, "clock_ghz") if args.operands == "randn" else None
    log(f"[bench] step {ms_step:.4f} ms (fused calls; as two timed launches {staged_ms:.4f} ms: prepare {prep_ms:.4f} "
        f"ms, attention {attn_ms:.4f} ms, median attention {float(np.median(t_attn)):.4f} ms); {value:.1f} TFLOP/s "
        f"step, {achieved:.1f} TFLOP/s attention kernel ({100 * achieved / PEAK_BF16_TFLOPS:.1f}% of bf16 peak); "
        f"wall {wall:.3f} s")

    result = {
        # BASELINE's metric for its own configuration; the other workloads name their shape
        "metric": METRIC if args.workload == "qwen-step" else
                  f"attention TFLOP/s + % bf16 MFMA peak; ms/call at {Sq} queries over {Sk} keys, {H}x128 "
                  f"({args.workload})",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "preroll": {"calls": pre_calls, "seconds": round(pre_s, 3),
                    "note": "untimed fused calls after the warm-up, the same for every --warmup"},
        "ms_per_step": round(ms_step, 5),
        "staged_ms_per_step": round(staged_ms, 5),
        "staged_note": "lr_joint_prepare (also copies the value rows into the workspace) + lr_joint_attention_images, "
                       "an event between the launches",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic" if args.operands == "randn" else "synthetic zeros (power study, not BASELINE's N(0,1))",
        "config": {"workload": f"{args.workload}-joint-attention", "batch": 1, "tokens": Sq, "keys": Sk,
                   "prefix_keys": n_pre, "text_tokens": w["n_text"], "heads": H, "head_dim": 128, "causal": False,
                   "qk_rmsnorm": True, "rope": w["kind"], "operands": "N(0,1)" if args.operands == "randn" else "zeros",
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic_from_profile(args.workload, KERNEL),
                     "kernel": KERNEL, "kernel_ms": round(attn_ms, 5),
                     "clock_ghz": clock,
                     "peak_at_clock": None if clock is None else round(PEAK_BF16_TFLOPS * clock / 2.4, 1)},
        "kernels_ms": {"prepare": round(prep_ms, 5), "attention": round(attn_ms, 5)},
        "flops_per_call": flops,
    }

    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    if not args.no_cpu_baseline:
        fl_row = 4.0 * Sk * 128 * H
        log("[bench] cpu baseline (oracle fp32 flash path, sampled query rows) ...")
        qb = q.cpu().view(torch.int16).numpy().view(np.uint16)
        kb = k.cpu().view(torch.int16).numpy().view(np.uint16)
        vb = v.cpu().view(torch.int16).numpy().view(np.uint16)
        cb = cpu_baseline(qb, kb, vb, cos_np, sin_np, Sq, H, fl_row, n_pre=n_pre)
        got = out.cpu().view(torch.int16).numpy().view(np.uint16)[cb["rows"]]
        gotf = (got.astype(np.uint32) << 16).view(np.float32)
        d = np.abs(gotf.astype(np.float64) - cb["out"])
        _, avail, model = host_cpus()
        rel = float(np.linalg.norm(gotf.astype(np.float64) - cb["out"]) / np.linalg.norm(cb["out"].astype(np.float64)))
        result["cpu_baseline"] = {"value": round(cb["value"], 4), "unit": "TFLOP/s", "cores": cb["threads"],
                                  "kind": "port", "host_cpus": avail, "cpu_model": model,
                                  "sample": f"{len(cb['rows'])} of {Sq} query rows x {H} heads over all {Sk} keys "
                                            f"(norm+rope+attention, fp32): median of {cb['runs']} runs, "
                                            f"{cb['seconds']:.2f} s each"}
        result["check"] = {"rows": int(len(cb["rows"])), "max_abs": float(d.max()), "mean_abs": float(d.mean()),
                           "rel_l2": rel, "bar": {"max_abs": 2e-2, "mean_abs": 2e-3, "rel_l2": 3e-3},
                           "pass": bool(d.max() <= 2e-2 and d.mean() <= 2e-3 and rel <= 3e-3)}
        log(f"[bench] cpu {cb['value']:.4f} TFLOP/s on {cb['threads']} threads; GPU vs CPU on sampled rows: "
            f"max-abs {d.max():.3e} mean-abs {d.mean():.3e}")
    print(json.dumps(result), flush=True)


def h3_table(S: int):
    """A bf16 H3 rotary table [S, 48, 2, 2] (rows [S, 192]) from H3's own layout arithmetic (rope.h3_positions /
    h3_rope_table: a text + video layout's positions, 16 frequencies per axis), tiled to S rows."""
    import numpy as np

    from localrouter_amd import rope
    pos = rope.h3_positions(24, 3, 8, 12, 15)
    inv = (1.0 / np.power(10000.0, np.arange(16) / 16.0)).astype(np.float32)
    tab = rope.h3_rope_table(pos, inv).reshape(-1, 192)
    return np.ascontiguousarray(np.tile(tab, (-(-S // tab.shape[0]), 1))[:S])


# H3's rmsRope arguments: rot 96 and the engine's eps 1e-5 (src/engines/minimax_h3/dit.zig:40, :665)
H3_ROT, H3_EPS = 96, 1e-5


def cpu_baseline_int8(qkv_bits, qn, kn, tab, S, H, budget_s=10.0):
    """The oracle's H3 chain (rmsRope in its bf16 rounding mode, anchor, rotation, quantisers, fp64 attention over the
    quantised operands) for a sample of heads and query rows, timed on host cores. Returns ops/s over the sampled
    rows and the outputs."""
    import numpy as np

    import oracle
    threads = host_cpus()[0]
    oracle.set_threads(threads)
    rng = np.random.default_rng(0)
    heads = [0, H // 2, H - 1]

    def rope(x, w):
        y = oracle.rms_rope(np.ascontiguousarray(x)[:, None, :], None, w_bf16=w, table_kind=oracle.TABLE_MAT2_BF16,
                            ta=tab, pairing=oracle.PAIR_SPLIT_HALF, rot=H3_ROT, eps=H3_EPS, round_norm=True)
        return oracle.f32_to_bf16(y[:, 0, :])

    def run(rows):
        t0 = time.perf_counter()
        outs = {}
        for h in heads:
            q, k, v = (np.ascontiguousarray(qkv_bits[:, i, h]) for i in range(3))
            q, k = rope(q, qn), rope(k, kn)
            rot = oracle.i8_rotation_for(S)
            a = oracle.i8_anchor(k)
            q8, qs = oracle.i8_quant_rows(q[rows], rot)
            k8, ks = oracle.i8_quant_rows(k, rot, a, oracle.I8_KGROUP)
            v8, vs = oracle.i8_quant_v(v)
            outs[h] = oracle.i8_attention(q8, qs, k8, ks, v8, vs)
        return time.perf_counter() - t0, outs

    ops_row = 4.0 * S * 128 * len(heads)
    probe = np.sort(rng.choice(S, size=64, replace=False))
    dt, _ = run(probe)
    n = int(min(S, max(64, budget_s / 3 * (64 * ops_row / dt) / ops_row)) // 32 * 32)
    rows = np.sort(rng.choice(S, size=n, replace=False))
    times, outs, spent = [], None, 0.0
    while spent < budget_s or len(times) < 3:
        dt, outs = run(rows)
        times.append(dt)
        spent += dt
    dt = float(np.median(times))
    return dict(value=n * ops_row / dt / 1e12, threads=threads, rows=rows, heads=heads, outs=outs, seconds=dt,
                runs=len(times))


def bench_int8(args):
    import numpy as np
    import torch

    from localrouter_amd import _lib, ops

    S, H = 5967, 56
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    L = _lib.load()
    rc = L.lr_attn_init()
    if rc != 0:
        raise SystemExit(f"lr_attn_init: {rc} (not a gfx950?)")
    log(f"[bench] workload h3-int8: S={S} H={H}, packed qkv [S, 3*H*128], rmsRope rot {H3_ROT}")
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    qkv = torch.randn((S, 3 * H * 128), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    qkv_u = qkv.clone()   # the unfused chain's buffer (its rmsRope works in place)
    qn = (1.0 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1.0 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
    tab_np = h3_table(S)
    tab = torch.from_numpy(tab_np.view(np.int16)).to(dev).view(torch.bfloat16)
    out = torch.empty((S, H * 128), dtype=torch.bfloat16, device=dev)
    ws_bytes = ops.int8_workspace_bytes(H, S)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    row = 3 * H * 128
    strides = (S * row, 128, row)

    def qkv_ptrs(t):
        return tuple(t.data_ptr() + i * H * 128 * 2 for i in range(3))

    q_ptr, k_ptr, v_ptr = qkv_ptrs(qkv)
    qu_ptr, ku_ptr, vu_ptr = qkv_ptrs(qkv_u)

    def prep_rope():   # Kitchen.rmsRope + Kitchen.attentionPrep, fused (qkv unmodified)
        _lib.call("lr_int8_attention_prep_rope", q_ptr, k_ptr, v_ptr, ws.data_ptr(), 1, H, H, S, S, 128, *strides,
                  *strides, *strides, qn.data_ptr(), kn.data_ptr(), tab.data_ptr(), 192, H3_ROT, H3_EPS, sh)

    def attn():
        _lib.call("lr_int8_attention_kernel", out.data_ptr(), ws.data_ptr(), 1, H, H, S, S, 128, ops.SCALE_128, 1, sh)

    def rms_rope_u():   # the unfused chain: Kitchen.rmsRope in place, then Kitchen.attentionPrep
        _lib.call("lr_rms_rope_qk_bf16", qu_ptr, ku_ptr, S, H, row, row, qn.data_ptr(), kn.data_ptr(), tab.data_ptr(),
                  192, H3_ROT, H3_EPS, sh)

    def prep_u():
        _lib.call("lr_int8_attention_prep", qu_ptr, ku_ptr, vu_ptr, ws.data_ptr(), 1, H, H, S, S, 128, *strides,
                  *strides, *strides, sh)

    def chain():
        prep_rope()
        attn()

    for _ in range(args.warmup):
        chain()
    torch.cuda.synchronize()
    pre_calls, pre_s = preroll(chain, args.preroll_s)
    log(f"[bench] warmup {args.warmup} done, pre-roll {pre_calls} chains in {pre_s:.2f} s; timing {args.steps} steps")
    K = args.steps

    def timed(fns):
        """K steps of the calls fns back to back: (ms per step from events around the loop, ms per call from events
        between the calls of a second loop)."""
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(K):
            for f in fns:
                f()
        e1.record(stream)
        torch.cuda.synchronize()
        step = e0.elapsed_time(e1) / K
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(fns) * K + 1)]
        torch.cuda.synchronize()
        for i in range(K):
            for j, f in enumerate(fns):
                ev[len(fns) * i + j].record(stream)
                f()
        ev[-1].record(stream)
        torch.cuda.synchronize()
        per = [float(np.mean([ev[len(fns) * i + j].elapsed_time(ev[len(fns) * i + j + 1]) for i in range(K)]))
               for j in range(len(fns))]
        return step, per

    t_wall = time.perf_counter()
    ms_step, (prep_ms, attn_ms) = timed([prep_rope, attn])
    wall = time.perf_counter() - t_wall
    got = out.cpu()
    # the engine's unfused chain on the same inputs, for comparison (and its output: the same bits)
    ms_unfused, (rope_u_ms, prep_u_ms, attn_u_ms) = timed([rms_rope_u, prep_u, attn])
    qkv_u.copy_(qkv)
    rms_rope_u()
    prep_u()
    attn()
    torch.cuda.synchronize()
    same = bool(torch.equal(out.cpu(), got))
    ops_call = 4.0 * S * S * 128 * H
    value = ops_call / (ms_step * 1e-3) / 1e12
    achieved = ops_call / (attn_ms * 1e-3) / 1e12
    log(f"[bench] step {ms_step:.4f} ms (fused rmsRope + prep {prep_ms:.4f} ms, attention {attn_ms:.4f} ms); "
        f"{value:.1f} TOP/s step, {achieved:.1f} TOP/s attention kernel ({100 * achieved / PEAK_INT8_TOPS:.1f}% of "
        f"int8 peak); unfused chain {ms_unfused:.4f} ms (rmsRope {rope_u_ms:.4f} + prep {prep_u_ms:.4f} + attention "
        f"{attn_u_ms:.4f} ms), same output bits: {same}; wall {wall:.3f} s")
    result = {
        "metric": "int8 attention TOP/s + % int8 MFMA peak; ms/call at 5967 tokens, 56x128 (MiniMax H3)",
        "value": round(value, 2),
        "unit": "TOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "preroll": {"calls": pre_calls, "seconds": round(pre_s, 3),
                    "note": "untimed chains after the warm-up, the same for every --warmup"},
        "ms_per_step": round(ms_step, 5),
        "unfused_ms_per_step": round(ms_unfused, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "h3-int8-attention", "batch": 1, "tokens": S, "heads": H, "head_dim": 128,
                   "causal": False, "input": "packed qkv [S, 3*H*128] bf16 ~ N(0,1), before rmsRope",
                   "rms_rope": {"rot": H3_ROT, "eps": H3_EPS, "weights": "bf16 1 + 0.1 N(0,1)",
                                "table": "bf16 [S, 48, 2, 2] of H3's layout arithmetic"},
                   "step": "lr_int8_attention_prep_rope (rmsRope + prep) then lr_int8_attention_kernel (rows out)",
                   "output": "rows [S, H*128]", "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                     "frac": round(achieved / PEAK_INT8_TOPS, 4), "traffic": traffic_from_profile("h3-int8", "i8_attn"),
                     "kernel": "i8_attn_kernel<128, 4>", "kernel_ms": round(attn_ms, 5)},
        "kernels_ms": {"prep_rope": round(prep_ms, 5), "attention": round(attn_ms, 5),
                       "unfused": {"rms_rope": round(rope_u_ms, 5), "prep": round(prep_u_ms, 5),
                                   "attention": round(attn_u_ms, 5)}},
        "fused_equals_unfused": same,
        "ops_per_call": ops_call,
    }
    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline (oracle H3 chain, sampled heads and query rows) ...")
        qb = qkv.cpu().view(torch.int16).numpy().view(np.uint16).reshape(S, 3, H, 128)
        qnb = qn.cpu().view(torch.int16).numpy().view(np.uint16)
        knb = kn.cpu().view(torch.int16).numpy().view(np.uint16)
        cb = cpu_baseline_int8(qb, qnb, knb, tab_np, S, H)
        gb = got.view(torch.int16).numpy().view(np.uint16).reshape(S, H, 128)
        d = np.concatenate([np.abs(((gb[cb["rows"], h].astype(np.uint32) << 16).view(np.float32)).astype(np.float64)
                                   - cb["outs"][h]).ravel() for h in cb["heads"]])
        result["cpu_baseline"] = {"value": round(cb["value"], 4), "unit": "TOP/s", "cores": cb["threads"],
                                  "kind": "port",
                                  "sample": f"{len(cb['rows'])} of {S} query rows x heads {cb['heads']} over all {S} "
                                            f"keys (rmsRope + anchor + quantisers + fp64 attention): median of "
                                            f"{cb['runs']} runs, {cb['seconds']:.2f} s each"}
        result["check"] = {"rows": int(len(cb["rows"])), "heads": cb["heads"], "max_abs": float(d.max()),
                           "mean_abs": float(d.mean()), "bar": {"max_abs": 2e-2, "mean_abs": 2e-3}}
        log(f"[bench] cpu {cb['value']:.4f} TOP/s on {cb['threads']} threads; GPU vs CPU on sampled rows: "
            f"max-abs {d.max():.3e} mean-abs {d.mean():.3e}")
    print(json.dumps(result), flush=True)


def bench_mmdit(args):
    import numpy as np
    import torch

    from localrouter_amd import _lib, mmdit, rope_host
    from oracle import mmdit as om

    n_txt, gh, gw, D, F = 512, 64, 64, 3072, 12288
    n_img = gh * gw
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    rc = _lib.load().lr_attn_init()
    if rc != 0:
        raise SystemExit(f"lr_attn_init: {rc} (not a gfx950?)")
    log(f"[bench] workload mmdit: {n_txt} text + {n_img} image tokens, hidden {D}, MLP {F}")
    w = mmdit.make_weights(D, F, dev, seed=args.seed, std=0.02)
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed + 1)
    txt0 = torch.randn((n_txt, D), generator=g, device=dev).to(torch.bfloat16)
    img0 = torch.randn((n_img, D), generator=g, device=dev).to(torch.bfloat16)
    c_np, s_np = rope_host.grid2d_table(n_txt, gh, gw)
    cos, sin = torch.from_numpy(c_np).to(dev), torch.from_numpy(s_np).to(dev)
    t = torch.tensor([0.5], dtype=torch.float32, device=dev)
    blk = mmdit.MMDiTBlock(w)
    blk.workspace(n_txt, n_img)
    blk.tune(n_txt, n_img)          # the fastest hipBLASLt candidate per GEMM shape (before anything is timed)
    stream = torch.cuda.current_stream()
    # one checked call on fresh copies (kept for the CPU comparison), then the timed calls in place
    txt_c, img_c = txt0.clone(), img0.clone()
    blk(txt_c, img_c, t, cos, sin)
    txt, img = txt0.clone(), img0.clone()
    for _ in range(args.warmup):
        blk(txt, img, t, cos, sin)
    torch.cuda.synchronize()
    pre_calls, pre_s = preroll(lambda: blk(txt, img, t, cos, sin), args.preroll_s)
    log(f"[bench] warmup {args.warmup} done, pre-roll {pre_calls} blocks in {pre_s:.2f} s; timing {args.steps} blocks")
    K = args.steps
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    e0.record(stream)
    for _ in range(K):
        blk(txt, img, t, cos, sin)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms_step = e0.elapsed_time(e1) / K
    flops = om.block_flops(n_txt, n_img, D, F)
    value = flops / (ms_step * 1e-3) / 1e12
    # the dominant kernel alone: the image stream's MLP up-projection GEMM
    x = torch.randn((n_img, D), generator=g, device=dev).to(torch.bfloat16)
    y = torch.empty((n_img, F), dtype=torch.bfloat16, device=dev)
    for _ in range(5):
        blk.linear(x, w["img.mlp_up"], y)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    ev[0].record(stream)
    for _ in range(20):
        blk.linear(x, w["img.mlp_up"], y)
    ev[1].record(stream)
    torch.cuda.synchronize()
    gemm_ms = ev[0].elapsed_time(ev[1]) / 20
    gemm_flops = 2.0 * n_img * F * D
    achieved = gemm_flops / (gemm_ms * 1e-3) / 1e12
    log(f"[bench] block {ms_step:.4f} ms = {value:.1f} TFLOP/s; MLP-up GEMM alone {gemm_ms:.4f} ms = "
        f"{achieved:.1f} TFLOP/s ({100 * achieved / PEAK_BF16_TFLOPS:.1f}% of bf16 peak); wall {wall:.3f} s")
    result = {
        "metric": "MMDiT block TFLOP/s; ms/block at 4096+512 tokens, hidden 3072, 24x128, MLP 12288",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "preroll": {"calls": pre_calls, "seconds": round(pre_s, 3),
                    "note": "untimed block calls after the warm-up, the same for every --warmup"},
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "mmdit-double-stream-block", "batch": 1, "text_tokens": n_txt, "image_tokens": n_img,
                   "hidden": D, "heads": D // 128, "mlp": F, "weights": "N(0, 0.02) bf16", "activations": "N(0, 1)",
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "kernel": "hipBLASLt GEMM 4096 x 12288 x 3072 (image MLP up-projection)",
                     "kernel_ms": round(gemm_ms, 5)},
        "flops_per_block": flops,
    }
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline (numpy fp32 oracle of the whole block) ...")
        bits = lambda a: a.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)  # noqa: E731
        wn = {k: (bits(v) if v.dtype == torch.bfloat16 else v.cpu().numpy()) for k, v in w.items()}
        tb, ib = bits(txt0), bits(img0)
        t0 = time.perf_counter()
        ref_t, ref_i = om.mmdit_block(tb, ib, wn, 0.5, c_np, s_np)
        cpu_s = time.perf_counter() - t0
        got = np.concatenate([bits(txt_c), bits(img_c)])
        got = (got.astype(np.uint32) << 16).view(np.float32)
        d = np.abs(got - np.concatenate([ref_t, ref_i]))
        result["cpu_baseline"] = {"value": round(flops / cpu_s / 1e12, 4), "unit": "TFLOP/s",
                                  "cores": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)),
                                  "kind": "port", "sample": f"one whole block (all {n_txt + n_img} rows, numpy fp32 "
                                                            f"BLAS GEMMs + the oracle's fp32 attention): {cpu_s:.2f} s"}
        result["check"] = {"rows": n_txt + n_img, "max_abs": float(d.max()), "mean_abs": float(d.mean()),
                           "bar": {"max_abs": 6.25e-2, "mean_abs": 2e-3}}
        log(f"[bench] cpu {flops / cpu_s / 1e12:.4f} TFLOP/s ({cpu_s:.2f} s); GPU vs oracle max-abs {d.max():.3e} "
            f"mean-abs {d.mean():.3e}")
    blk.close()
    print(json.dumps(result), flush=True)



# Kandinsky-6's flash-dispatched attention shapes (src/engines/kandinsky6/dit/launch.zig:260-300): (name, queries, keys,
# heads); q, k, v and out are rows of heads x 128 (row stride 4096 for 32 heads, 2048 for 16)
K6_SHAPES = [("visual-self", 50220, 50220, 32), ("video-from-audio", 50220, 218, 32),
             ("audio-from-video", 218, 50220, 16), ("audio-self", 218, 218, 16)]


def bench_k6(args):
    import numpy as np
    import torch

    from localrouter_amd import _lib, ops

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    L = _lib.load()
    rc = L.lr_attn_init()
    if rc != 0:
        raise SystemExit(f"lr_attn_init: {rc} (not a gfx950?)")
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    scale = ops.SCALE_128
    ws_bytes = max(ops.attention_ws_bytes(W, H, S) for _, W, S, H in K6_SHAPES)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    calls = []
    for name, W, S, H in K6_SHAPES:
        q = torch.randn((W, H, 128), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        k = torch.randn((S, H, 128), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        v = torch.randn((S, H, 128), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        out = torch.empty_like(q)
        rs = H * 128
        argv = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), 0, W, H, H, S, 0, scale, rs, rs, rs,
                ws.data_ptr(), ws_bytes, sh)
        calls.append(dict(name=name, W=W, S=S, H=H, q=q, k=k, v=v, out=out, argv=argv,
                          flops=4.0 * W * S * 128 * H))
        log(f"[bench] k6 {name}: {W} queries over {S} keys, {H} heads; workspace route "
            f"{'split/stream' if ops.attention_ws_bytes(W, H, S) else 'plain'}")

    def run(c):
        _lib.call("lr_attention_bf16_ws", *c["argv"])

    def step():
        for c in calls:
            run(c)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    pre_calls, pre_s = preroll(step, args.preroll_s)
    log(f"[bench] warmup {args.warmup} done, pre-roll {pre_calls} steps in {pre_s:.2f} s; timing {args.steps} steps")

    K = args.steps
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    e0.record(stream)
    for _ in range(K):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms_step = e0.elapsed_time(e1) / K
    # the same steps with an event between the calls: each shape's time
    n = len(calls)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n * K + 1)]
    torch.cuda.synchronize()
    for i in range(K):
        for j, c in enumerate(calls):
            ev[n * i + j].record(stream)
            run(c)
    ev[n * K].record(stream)
    torch.cuda.synchronize()
    per = {c["name"]: float(np.mean([ev[n * i + j].elapsed_time(ev[n * i + j + 1]) for i in range(K)]))
           for j, c in enumerate(calls)}
    flops = sum(c["flops"] for c in calls)
    value = flops / (ms_step * 1e-3) / 1e12
    vis = calls[0]
    achieved = vis["flops"] / (per[vis["name"]] * 1e-3) / 1e12
    clock = from_profile("k6", KERNEL, "clock_ghz")
    log(f"[bench] step {ms_step:.4f} ms = {value:.1f} TFLOP/s; " + ", ".join(
        f"{c['name']} {per[c['name']]:.4f} ms ({c['flops'] / (per[c['name']] * 1e-3) / 1e12:.1f} TFLOP/s)"
        for c in calls) + f"; visual self-attention {100 * achieved / PEAK_BF16_TFLOPS:.1f}% of bf16 peak; "
        f"wall {wall:.3f} s")
    result = {
        "metric": "K6 attention TFLOP/s + % bf16 MFMA peak; ms per step of the four Kandinsky-6 attention shapes",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "preroll": {"calls": pre_calls, "seconds": round(pre_s, 3),
                    "note": "untimed steps after the warm-up, the same for every --warmup"},
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "k6-attention", "shapes": [dict(name=c["name"], queries=c["W"], keys=c["S"],
                                                                 heads=c["H"]) for c in calls],
                   "head_dim": 128, "causal": False, "operands": "N(0,1)", "entry_point": "lr_attention_bf16_ws",
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic_from_profile("k6", KERNEL),
                     "kernel": KERNEL + "<true> (visual self-attention)", "kernel_ms": round(per[vis["name"]], 5),
                     "clock_ghz": clock,
                     "peak_at_clock": None if clock is None else round(PEAK_BF16_TFLOPS * clock / 2.4, 1)},
        "calls_ms": {c["name"]: round(per[c["name"]], 5) for c in calls},
        "flops_per_step": flops,
    }

    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    if not args.no_cpu_baseline:
        import oracle
        log("[bench] cpu baseline (oracle fp32 flash path, sampled query rows of the visual self-attention) ...")
        threads, avail, model = host_cpus()
        oracle.set_threads(threads)
        f32 = lambda t: oracle.bf16_to_f32(t.cpu().view(torch.int16).numpy().view(np.uint16))
        qf, kf, vf = f32(vis["q"]), f32(vis["k"]), f32(vis["v"])
        W, fl_row = vis["W"], 4.0 * vis["S"] * 128 * vis["H"]
        rng = np.random.default_rng(0)

        def cpu(rows):
            t0 = time.perf_counter()
            o = oracle.attention(qf, kf, vf, scale=scale, precise=False, rows=rows)
            return time.perf_counter() - t0, o

        dt, _ = cpu(np.sort(rng.choice(W, size=32, replace=False)))
        nrows = int(min(W, max(32, 10.0 / 3 * 32 / dt)) // 32 * 32)
        rows = np.sort(rng.choice(W, size=nrows, replace=False))
        times, ref, spent = [], None, 0.0
        while spent < 10.0 or len(times) < 3:
            dt, ref = cpu(rows)
            times.append(dt)
            spent += dt
        dt = float(np.median(times))
        got = f32(vis["out"])[rows].astype(np.float64)
        d = np.abs(got - ref)
        rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref.astype(np.float64)))
        result["cpu_baseline"] = {"value": round(nrows * fl_row / dt / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
                                  "kind": "port", "host_cpus": avail, "cpu_model": model,
                                  "sample": f"{nrows} of {W} query rows x {vis['H']} heads of the visual "
                                            f"self-attention over all {vis['S']} keys (fp32 flash path): median of "
                                            f"{len(times)} runs, {dt:.2f} s each"}
        result["check"] = {"rows": nrows, "max_abs": float(d.max()), "mean_abs": float(d.mean()), "rel_l2": rel,
                           "bar": {"max_abs": 2e-2, "mean_abs": 2e-3, "rel_l2": 3e-3},
                           "pass": bool(d.max() <= 2e-2 and d.mean() <= 2e-3 and rel <= 3e-3)}
        log(f"[bench] cpu {result['cpu_baseline']['value']:.4f} TFLOP/s on {threads} threads; GPU vs CPU on sampled "
            f"rows: max-abs {d.max():.3e} mean-abs {d.mean():.3e} rel-L2 {rel:.3e}")
    print(json.dumps(result), flush=True)



def bench_rows(args):
    import numpy as np
    import torch

    from localrouter_amd import _lib, ops

    S, H = 4608, 24
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    rc = _lib.load().lr_attn_init()
    if rc != 0:
        raise SystemExit(f"lr_attn_init: {rc} (not a gfx950?)")
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    q, k, v = (torch.randn((S, H, 128), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
               for _ in range(3))
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    scale, rs = ops.SCALE_128, H * 128
    ws_bytes = ops.attention_ws_bytes(S, H, S)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    log(f"[bench] workload rows: {S} queries over {S} keys, {H} heads (Ops.attention drop-in, rows in and out)")

    def ex(cfg):
        return lambda: _lib.call("lr_attention_bf16_ex", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), 0,
                                 S, H, H, S, 0, scale, rs, rs, rs, rs, 128, 128, cfg, sh)

    plain = lambda: _lib.call("lr_attention_bf16", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), 0, S, H,
                              H, S, 0, scale, rs, rs, rs, sh)
    variants = {"lr_attention_bf16_ws": lambda: _lib.call(
                    "lr_attention_bf16_ws", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), 0, S, H, H, S, 0,
                    scale, rs, rs, rs, ws.data_ptr(), ws_bytes, sh),
                "PIPE_W8": ex(ops.CFG_PIPE_W8), "PIPE_W4": ex(ops.CFG_PIPE_W4), "STREAM_W8": ex(ops.CFG_STREAM_W8)}

    def timed(call, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(n):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    for _ in range(args.warmup):
        plain()
        for f in variants.values():
            f()
    torch.cuda.synchronize()
    pre_calls, pre_s = preroll(plain, args.preroll_s)
    log(f"[bench] warmup {args.warmup} done, pre-roll {pre_calls} calls in {pre_s:.2f} s; timing {args.steps} steps")
    K = args.steps
    t_wall = time.perf_counter()
    ms_step = timed(plain, K)
    wall = time.perf_counter() - t_wall
    ref = out.clone()
    var_ms = {}
    for name, f in variants.items():
        preroll(f, 0.2)
        var_ms[name] = timed(f, K)
    # every route computes the same softmax: the outputs agree to bf16 rounding (checked loosely here; the parity tests
    # hold the oracle bars)
    same = {}
    for name, f in variants.items():
        f()
        torch.cuda.synchronize()
        same[name] = float((out.float() - ref.float()).abs().max())
    plain()
    torch.cuda.synchronize()
    flops = 4.0 * S * S * 128 * H
    value = flops / (ms_step * 1e-3) / 1e12
    clock = from_profile("rows", KERNEL, "clock_ghz")
    log(f"[bench] step {ms_step:.4f} ms = {value:.1f} TFLOP/s ({100 * value / PEAK_BF16_TFLOPS:.1f}% of bf16 peak, "
        f"lr_attention_bf16, AUTO); " + ", ".join(f"{n} {t:.4f} ms" for n, t in var_ms.items())
        + f"; max-abs difference to AUTO's output {max(same.values()):.3e}; wall {wall:.3f} s")
    result = {
        "metric": "attention TFLOP/s + % bf16 MFMA peak; ms/call of the Ops.attention drop-in (lr_attention_bf16, "
                  "rows in and out) at 4608 tokens, 24x128",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "preroll": {"calls": pre_calls, "seconds": round(pre_s, 3),
                    "note": "untimed calls after the warm-up, the same for every --warmup"},
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "rows-attention", "batch": 1, "tokens": S, "keys": S, "heads": H, "head_dim": 128,
                   "causal": False, "qk_rmsnorm": False, "rope": None, "operands": "N(0,1)",
                   "entry_point": "lr_attention_bf16 (AUTO)", "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(value, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(value / PEAK_BF16_TFLOPS, 4), "traffic": traffic_from_profile("rows", KERNEL),
                     "kernel": KERNEL + "<true> (AUTO at this shape: whole 256-query blocks over the key rows)",
                     "kernel_ms": round(ms_step, 5), "clock_ghz": clock,
                     "peak_at_clock": None if clock is None else round(PEAK_BF16_TFLOPS * clock / 2.4, 1)},
        "variants_ms": {n: round(t, 5) for n, t in var_ms.items()},
        "variants_max_abs_vs_auto": same,
        "flops_per_call": flops,
    }

    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    if not args.no_cpu_baseline:
        import oracle
        log("[bench] cpu baseline (oracle fp32 flash path, sampled query rows) ...")
        threads, avail, model = host_cpus()
        oracle.set_threads(threads)
        f32 = lambda t: oracle.bf16_to_f32(t.cpu().view(torch.int16).numpy().view(np.uint16))
        qf, kf, vf = f32(q), f32(k), f32(v)
        fl_row = 4.0 * S * 128 * H
        rng = np.random.default_rng(0)

        def cpu(rows):
            t0 = time.perf_counter()
            o = oracle.attention(qf, kf, vf, scale=scale, precise=False, rows=rows)
            return time.perf_counter() - t0, o

        dt, _ = cpu(np.sort(rng.choice(S, size=64, replace=False)))
        nrows = int(min(S, max(64, 10.0 / 3 * 64 / dt)) // 32 * 32)
        rows = np.sort(rng.choice(S, size=nrows, replace=False))
        times, ref_cpu, spent = [], None, 0.0
        while spent < 10.0 or len(times) < 3:
            dt, ref_cpu = cpu(rows)
            times.append(dt)
            spent += dt
        dt = float(np.median(times))
        got = f32(out)[rows].astype(np.float64)
        d = np.abs(got - ref_cpu)
        rel = float(np.linalg.norm(got - ref_cpu) / np.linalg.norm(ref_cpu.astype(np.float64)))
        result["cpu_baseline"] = {"value": round(nrows * fl_row / dt / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
                                  "kind": "port", "host_cpus": avail, "cpu_model": model,
                                  "sample": f"{nrows} of {S} query rows x {H} heads over all {S} keys (fp32 flash "
                                            f"path): median of {len(times)} runs, {dt:.2f} s each"}
        result["check"] = {"rows": nrows, "max_abs": float(d.max()), "mean_abs": float(d.mean()), "rel_l2": rel,
                           "bar": {"max_abs": 2e-2, "mean_abs": 2e-3, "rel_l2": 3e-3},
                           "pass": bool(d.max() <= 2e-2 and d.mean() <= 2e-3 and rel <= 3e-3)}
        log(f"[bench] cpu {result['cpu_baseline']['value']:.4f} TFLOP/s on {threads} threads; GPU vs CPU on sampled "
            f"rows: max-abs {d.max():.3e} mean-abs {d.mean():.3e} rel-L2 {rel:.3e}")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
