"""Graph capture of the library's calls: lr_joint_attention_fused, lr_joint_attention_fused_noalloc (after
lr_attn_init), lr_attention_bf16_ws (the streaming kernel over key rows with its split tail, and the key split of a
few-query call), lr_int8_attention_rows and lr_mmdit_block_bf16 recorded into one HIP graph (torch.cuda.CUDAGraph)
and replayed, each replay compared bit for bit with the same calls made eagerly.

The reference records whole denoising steps the same way and falls back to eager launches when capture fails
(src/engines/qwen_image/dit.zig:469-484, src/engines/minimax_h3/dit.zig:557-577). The library's calls neither
synchronise nor allocate and issue no memset (the split tail's arrival counters are cleared by the preparation
kernel, or over key rows by a one-workgroup fill kernel), so the captured graph holds kernels only. Between the replays the program does eager work of its own (the
outputs are cleared with torch's fill kernel, the MMDiT streams restored) and synchronises; every replay must give
the eager bits."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests._util import from_dev, to_dev

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from localrouter_amd import _lib, mmdit, ops, rope_host  # noqa: E402


def _fused_args(q, k, v, out, cos, sin, Sq, Sk, H, HK):
    rs_q, rs_k, rs_o = H * 128, HK * 128, H * 128
    return (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), None, None, ops.TABLE_COSSIN_F32,
            cos.data_ptr(), sin.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.stride(0), ops.PAIR_INTERLEAVED, 128,
            1e-6, Sq, Sk, H, HK, 0, 0, ops.SCALE_128, rs_q, rs_k, rs_k, rs_o, 0)


def test_graph_capture_replays_equal_eager():
    L = _lib.load()
    assert L.lr_attn_init() == 0
    dev = torch.device("cuda", 0)
    # joint attention: cfg1's 256 text + 32x32 image tokens at 4 heads (every block a cut tail block, so the replay
    # also exercises the split tail's partials and arrival counters)
    H = 4
    cos_np, sin_np = rope_host.grid2d_table(256, 32, 32)
    S = cos_np.shape[0]
    q, k, v = (to_dev(oracle.synth_bf16(11, i, (S, H, 128))) for i in (1, 2, 3))
    cos, sin = torch.from_numpy(cos_np).to(dev), torch.from_numpy(sin_np).to(dev)
    ws = torch.empty(ops.workspace_bytes(S, H), dtype=torch.uint8, device=dev)
    # INT8 chain: packed qkv of 300 tokens x 4 heads, rows output
    Si, Hi = 300, 4
    qkv = to_dev(oracle.synth_bf16(12, 1, (Si, 3 * Hi * 128)))
    ws8 = torch.empty(ops.int8_workspace_bytes(Hi, Si), dtype=torch.uint8, device=dev)
    # attention over rows with a workspace: 1,280 queries x 8 heads over 4,096 keys (40 query blocks: the streaming
    # kernel over key rows, its split tail's partials and counters in the workspace) and 218 x 4 heads over 2,000 keys
    # (4 query blocks: split over the keys, then merged)
    rows_cases = [(1280, 8, 4096), (218, 4, 2000)]
    rows_in = [tuple(to_dev(oracle.synth_bf16(13 + i, j, (nk if j else W, Hr, 128))) for j in (0, 1, 2))
               for i, (W, Hr, nk) in enumerate(rows_cases)]
    rows_ws = [torch.empty(ops.attention_ws_bytes(W, Hr, nk), dtype=torch.uint8, device=dev) for W, Hr, nk in rows_cases]
    assert rows_ws[0].numel() == 69207040 and 0 < rows_ws[1].numel() != 69207040
    # MMDiT block: 16 text + 6x8 image rows, hidden 256 (2 heads), MLP 512
    Dm, Fm, n_txt, gh, gw = 256, 512, 16, 6, 8
    wts = mmdit.make_weights(Dm, Fm, dev, seed=3, std=0.05)
    blk = mmdit.MMDiTBlock(wts)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    txt0 = torch.randn((n_txt, Dm), generator=g, device=dev).to(torch.bfloat16)
    img0 = torch.randn((gh * gw, Dm), generator=g, device=dev).to(torch.bfloat16)
    mcos_np, msin_np = rope_host.grid2d_table(n_txt, gh, gw)
    mcos, msin = torch.from_numpy(mcos_np).to(dev), torch.from_numpy(msin_np).to(dev)
    tt = torch.tensor([0.3], dtype=torch.float32, device=dev)

    outs = {name: torch.empty_like(q) for name in ("fused", "noalloc")}
    for i, (qr, _, _) in enumerate(rows_in):
        outs[f"rows{i}"] = torch.empty_like(qr)
    out8 = torch.empty((Si, Hi * 128), dtype=torch.bfloat16, device=dev)
    txt, img = txt0.clone(), img0.clone()

    def calls():
        sh = torch.cuda.current_stream().cuda_stream
        assert L.lr_joint_attention_fused(*_fused_args(q, k, v, outs["fused"], cos, sin, S, S, H, H), ws.data_ptr(),
                                          ws.numel(), sh) == 0
        assert L.lr_joint_attention_fused_noalloc(*_fused_args(q, k, v, outs["noalloc"], cos, sin, S, S, H, H),
                                                  sh) == 0
        for i, (qr, kr, vr) in enumerate(rows_in):
            ops.attention_ws(qr, kr, vr, outs[f"rows{i}"], workspace=rows_ws[i])
        ops.kitchen_attention(qkv, Hi, out=out8, workspace=ws8, rows=True)
        blk(txt, img, tt, mcos, msin)

    # eager: the reference bits (the block plans its GEMMs and takes its workspace here, before any capture)
    calls()
    torch.cuda.synchronize()
    eager = {n: from_dev(t) for n, t in outs.items()}
    eager["int8"] = from_dev(out8)
    eager["txt"], eager["img"] = from_dev(txt), from_dev(img)
    assert np.array_equal(eager["fused"], eager["noalloc"])

    def reset():
        for t in (*outs.values(), out8):
            t.zero_()
        txt.copy_(txt0)
        img.copy_(img0)

    reset()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls()
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"[graph] replay {rep}", flush=True)
        reset()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = {n: from_dev(t) for n, t in outs.items()}
        got["int8"] = from_dev(out8)
        got["txt"], got["img"] = from_dev(txt), from_dev(img)
        for n in eager:
            assert np.array_equal(got[n], eager[n]), f"replay {rep}: {n} differs from the eager call"
        # eager work of the program's own between replays
        (q.float() * 2).sum().item()
    graph.reset()
    blk.close()
