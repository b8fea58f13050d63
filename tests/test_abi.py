"""The C ABI library on the CPU: it loads, exports exactly what include/lr_attn.h declares, and rejects bad arguments
with hipErrorInvalidValue before touching the GPU (no compute calls here)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from localrouter_amd import _lib, ops
from tests._util import img_index

HIP_ERROR_INVALID_VALUE = 1


def _declared():
    text = _lib.HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(?:int|size_t)\s+(lr_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    declared = _declared()
    assert len(declared) >= 10
    for name in declared:
        assert hasattr(L, name), f"{name} declared in lr_attn.h but not exported"
    assert sorted(_lib.SIGNATURES) == declared, "ctypes signatures out of sync with lr_attn.h"


def test_abi_version():
    header = _lib.HEADER.read_text()
    declared = int(re.search(r"#define LR_ATTN_ABI_VERSION (\d+)", header).group(1))
    assert _lib.load().lr_attn_abi_version() == declared == 9


def test_workspace_bytes():
    L = _lib.load()
    # key tile images then value tile images, [HK][ceil(Sk/64)] x 16 KB each, then the split area: two partial slots
    # of 8 waves x (64 x 64 fp32 O + 64 x (m, l)) for each of at most 256 workgroups, then 256 int counters
    header = _lib.HEADER.read_text()
    split = int(re.search(r"#define LR_JOINT_SPLIT_BYTES \(\(size_t\)(\d+)\)", header).group(1))
    assert split == 2 * 256 * 8 * (64 * 64 * 4 + 64 * 8) + 4 * 256
    assert L.lr_joint_attention_workspace_bytes(4608, 24) == 2 * 24 * 72 * 16384 + split
    assert L.lr_joint_attention_workspace_bytes(3, 1) == 2 * 16384 + split
    assert L.lr_joint_attention_workspace_bytes(65, 2) == 2 * 2 * 2 * 16384 + split
    assert ops.workspace_bytes(65, 2) == 2 * 2 * 2 * 16384 + split
    assert L.lr_joint_attention_workspace_bytes(0, 24) == 0
    assert "SK_AREA" not in header and "#define LR_ATTN_CFG_STREAM_W8 9" in header


# fake, well-aligned device addresses: validation must reject before any HIP call is made
A = 0x10000
W = 0x100000   # a fake workspace address past every fake tensor
SPLIT = 69207040   # LR_JOINT_SPLIT_BYTES


@pytest.mark.parametrize("args,why", [
    ((0, A, A, A, 0, 8, 2, 2, 8, 0, 0.088, 256, 256, 256, None), "null q"),
    ((A, A, A, A, 0, 8, 2, 2, 0, 0, 0.088, 256, 256, 256, None), "nkeys 0"),
    ((A, A, A, A, 0, 0, 2, 2, 8, 0, 0.088, 256, 256, 256, None), "W 0"),
    ((A, A, A, A, 0, 8, 3, 2, 8, 0, 0.088, 384, 256, 384, None), "H % HK"),
    ((A + 2, A, A, A, 0, 8, 2, 2, 8, 0, 0.088, 256, 256, 256, None), "misaligned q"),
    ((A, A, A, A, 0, 8, 2, 2, 8, 0, 0.088, 260, 256, 256, None), "row stride not 16-byte"),
    ((A, A, A, A, 0, 8, 2, 2, 8, 0, 0.088, 128, 256, 256, None), "row stride narrower than the heads"),
    ((A, A, A, A, 0, 8, 2, 2, 8, 0, -1.0, 256, 256, 256, None), "negative scale"),
    ((A, A, A, A, 0, 8, 2, 2, 8, 0, float("inf"), 256, 256, 256, None), "infinite scale"),
    ((A, A, A, A, -1, 8, 2, 2, 8, 1, 0.088, 256, 256, 256, None), "negative p0"),
    ((A, A, A, A, 0, 8, 2, 2, 8, 2, 0.088, 256, 256, 256, None), "causal not 0/1"),
])
def test_attention_rejects(args, why):
    assert _lib.load().lr_attention_bf16(*args) == HIP_ERROR_INVALID_VALUE, why


def test_attention_ex_rejects_bad_config():
    L = _lib.load()
    assert L.lr_attention_bf16_ex(A, A, A, A, 0, 8, 2, 2, 8, 0, 0.088, 256, 256, 256, 256, 128, 128, 99,
                                  None) == HIP_ERROR_INVALID_VALUE


def _fused(**kw):
    a = dict(q=A, k=A, v=A, out=A, wq=None, wk=None, kind=1, qa=A, qb=A, ka=A, kb=A, ts=64, pairing=0, rot=128,
             eps=1e-6, Sq=8, Sk=8, H=2, HK=2, p0=0, causal=0, scale=0.088, qrs=256, krs=256, vrs=256, ors=256, n_pre=0,
             ws=W, wsb=2 * 2 * 16384 + SPLIT, config=0, stream=None)
    a.update(kw)
    return _lib.load().lr_joint_attention_fused_ex(*a.values())


@pytest.mark.parametrize("kw,why", [
    (dict(ws=0), "no workspace"),
    (dict(ws=A + 16), "workspace not 256-aligned"),
    (dict(wsb=100), "workspace too small"),
    (dict(wsb=2 * 16384 + SPLIT), "workspace short of the value images"),
    (dict(wsb=2 * 2 * 16384), "workspace holds the images but not the split area"),
    (dict(ws=A + 256), "out overlaps the workspace"),
    (dict(out=A + 0x1000, k=A + 0x1000), "out overlaps k_raw"),
    (dict(out=A + 0x1000, v=A + 0x1100), "out overlaps v"),
    (dict(ors=(1 << 23) + 8), "out row stride beyond 2^23"),
    (dict(ors=1 << 23), "out row stride 2^23: a block's 256 rows would span 4 GiB, past the 32-bit buffer range"),
    (dict(q=W), "q_raw overlaps the workspace the preparation writes"),
    (dict(k=W + 4096), "k_raw overlaps the workspace"),
    (dict(v=W + 4096), "v overlaps the workspace"),
    (dict(config=1), "plain-attention configuration on the fused call"),
    (dict(kind=7), "table kind"),
    (dict(pairing=1, rot=48), "split-half rot not a multiple of 32"),
    (dict(rot=130), "rot > 128"),
    (dict(rot=63), "odd rot"),
    (dict(qb=0), "cos/sin table without sin"),
    (dict(ts=10), "table stride below rot/2"),
    (dict(n_pre=9), "n_pre > Sk"),
    (dict(eps=-1.0), "negative eps"),
    (dict(kind=2, ts=254), "bf16 2x2 table stride not a multiple of 4"),
])
def test_fused_rejects(kw, why):
    assert _fused(**kw) == HIP_ERROR_INVALID_VALUE, why


def test_stage_entry_points_reject():
    L = _lib.load()
    wsb = L.lr_joint_attention_workspace_bytes(8, 2)
    kv = dict(k=A, krs=256, v=A, vrs=256, wk=None, kind=1, ka=A, kb=A, ts=64, pairing=0, rot=128, eps=1e-6, Sk=8, HK=2,
              n_pre=0, ws=W, wsb=wsb, stream=None)

    def kv_call(**kw):
        a = dict(kv)
        a.update(kw)
        return L.lr_joint_kv_prepare(*a.values())

    assert kv_call(v=0) == HIP_ERROR_INVALID_VALUE              # the values are part of the prepared workspace
    assert kv_call(wsb=wsb - 2) == HIP_ERROR_INVALID_VALUE
    assert kv_call(vrs=200) == HIP_ERROR_INVALID_VALUE
    assert kv_call(k=W + 256) == HIP_ERROR_INVALID_VALUE          # k_raw inside the workspace it writes
    assert kv_call(v=W + 4096) == HIP_ERROR_INVALID_VALUE         # v inside the workspace
    pr = dict(q=A, ws=W, wsb=wsb, out=A, wq=None, kind=1, qa=A, qb=A, ts=64, pairing=0, rot=128, eps=1e-6, Sq=8, Sk=8,
              H=2, HK=2, p0=0, causal=0, scale=0.088, qrs=256, ors=256, config=0, stream=None)

    def pr_call(**kw):
        a = dict(pr)
        a.update(kw)
        return L.lr_joint_attention_prepared(*a.values())

    for cfg in (1, 2, 3, 8, 99):                                # only AUTO and STREAM_W8 read tile images
        assert pr_call(config=cfg) == HIP_ERROR_INVALID_VALUE, cfg
    assert pr_call(wsb=wsb - 256) == HIP_ERROR_INVALID_VALUE
    assert pr_call(ws=A + 256) == HIP_ERROR_INVALID_VALUE       # out overlaps the workspace


def test_rms_rope_rejects():
    L = _lib.load()
    ok = dict(src=A, srs=256, off=0, dst=A, drs=256, n=4, b=1, sbs=0, dbs=0, heads=2, w=None, wk=0, kind=1, ta=A,
              tb=A, ts=64, rot=128, pairing=0, eps=1e-6, rn=0, stream=None)

    def call(**kw):
        a = dict(ok)
        a.update(kw)
        return L.lr_rms_rope_bf16(*a.values())

    assert call(n=0) == HIP_ERROR_INVALID_VALUE
    assert call(off=3) == HIP_ERROR_INVALID_VALUE
    assert call(wk=1) == HIP_ERROR_INVALID_VALUE          # weight kind without a weight
    assert call(pairing=1, rot=40) == HIP_ERROR_INVALID_VALUE
    assert call(rn=2) == HIP_ERROR_INVALID_VALUE
    assert L.lr_rms_rope_qk_bf16(A, A, 4, 2, 768, 768, None, A, A, 192, 96, 1e-5, None) == HIP_ERROR_INVALID_VALUE


def _i8_plan(B, H, HK, Sq, Sk, d=128):
    """The INT8 workspace layout, restated: parts in order, each starting on a 256-byte boundary."""
    cta = 128 if Sk > 1024 and d == 128 else 64
    nt = -(-Sk // cta)
    skp, nvc = nt * cta, -(-Sk // 256)
    # the attention's split pieces: up to 4 per query block of 256 rows, 256 in all, none below 16 key tiles; rows of
    # d + 2 fp32
    pieces = min(4 * B * H * -(-Sq // 256), 256) if nt >= 16 else 0
    parts = [B * H * Sq * d, B * HK * skp * d, B * HK * skp * d, B * HK * nt * 1024, B * H * Sq * 4,
             B * HK * d * 4, B * HK * nvc * d * 4, B * HK * 4, B * HK * d * 2, pieces * 256 * (d + 2) * 4]
    return sum(-(-p // 256) * 256 for p in parts)


def test_int8_workspace_bytes():
    L = _lib.load()
    for args in ((1, 56, 56, 5967, 5967), (1, 2, 2, 80, 80), (2, 4, 2, 300, 1100), (1, 3, 1, 1, 1), (1, 2, 2, 1024, 1024),
                 (1, 2, 2, 1025, 1025)):
        assert L.lr_int8_attention_workspace_bytes(*args, 128) == _i8_plan(*args), args
    # head dim 64 (kitchen_launch.cu:196-241): 64-key tiles at every length, e.g. the gate's 1797 tokens x 32 heads
    for args in ((1, 32, 32, 1797, 1797), (1, 2, 2, 80, 80), (2, 4, 2, 300, 1100)):
        assert L.lr_int8_attention_workspace_bytes(*args, 64) == _i8_plan(*args, 64), args
    for d in (32, 96, 256):
        assert L.lr_int8_attention_workspace_bytes(1, 2, 2, 8, 8, d) == 0, d
    assert L.lr_int8_attention_workspace_bytes(1, 3, 2, 8, 8, 128) == 0      # H % HK
    assert L.lr_int8_attention_workspace_bytes(0, 2, 2, 8, 8, 128) == 0


def test_int8_rejects():
    L = _lib.load()
    ok = dict(q=A, k=A, v=A, o=A, ws=0x100000, B=1, H=2, HK=2, Sq=8, Sk=8, D=128, q_sb=0, q_sh=768, q_sn=768 * 2,
              k_sb=0, k_sh=768, k_sn=768 * 2, v_sb=0, v_sh=768, v_sn=768 * 2, scale=0.088, stream=None)

    def call(fn="lr_int8_attention", **kw):
        a = dict(ok)
        a.update(kw)
        return getattr(L, fn)(*a.values())

    for kw, why in ((dict(D=96), "head dim"), (dict(H=3), "H % HK"), (dict(q=A + 8), "misaligned q"),
                    (dict(k_sn=100), "stride not a multiple of 8"), (dict(ws=A + 16), "workspace alignment"),
                    (dict(ws=0), "no workspace"), (dict(scale=0.0), "scale"), (dict(Sk=0), "empty"),
                    (dict(o=A + 2), "misaligned out")):
        assert call(**kw) == HIP_ERROR_INVALID_VALUE, why
    assert call("lr_int8_attention_rows", B=2, q_sb=8 * 768) == HIP_ERROR_INVALID_VALUE  # rows: B 1 only
    d64 = dict(H=32, HK=32, Sq=1797, Sk=1797, D=64, q_sh=64, q_sn=3 * 32 * 64, k_sh=64, k_sn=3 * 32 * 64, v_sh=64,
               v_sn=3 * 32 * 64)
    assert call(**dict(d64, D=96)) == HIP_ERROR_INVALID_VALUE             # only 64 and 128
    assert call(**dict(d64, k_sn=100)) == HIP_ERROR_INVALID_VALUE          # head dim 64 keeps the stride rule
    assert L.lr_int8_attention_kernel(A, 0x100000, 1, 2, 2, 8, 8, 128, 0.088, 2, None) == HIP_ERROR_INVALID_VALUE
    # a workspace overlapping q, k, v (written by the prep while they are read) or out (read while out is written)
    for name in ("q", "k", "v", "o"):
        far = dict(q=1 << 40, k=2 << 40, v=3 << 40, o=4 << 40)
        assert call(**far, ws=far[name] + 256) == HIP_ERROR_INVALID_VALUE, name
    assert L.lr_int8_attention_kernel(0x100000 + 4096, 0x100000, 1, 2, 2, 8, 8, 128, 0.088, 1,
                                      None) == HIP_ERROR_INVALID_VALUE
    assert L.lr_int8_attention_prep(A, A, A, A + 64, 1, 2, 2, 8, 8, 128, 0, 768, 1536, 0, 768, 1536, 0, 768, 1536,
                                    None) == HIP_ERROR_INVALID_VALUE


def test_ops_has_no_cpu_path():
    """The torch-facing layer refuses CPU tensors instead of computing anything itself."""
    torch = pytest.importorskip("torch")
    from localrouter_amd import ops
    q = torch.zeros((4, 1, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ops.attention(q, q, q)


def test_mmdit_abi_on_cpu():
    """include/lr_mmdit.h: exports, workspace sizes and argument rejection (no GPU call is reached)."""
    import ctypes

    from localrouter_amd import mmdit
    text = re.sub(r"/\*.*?\*/", "", mmdit.HEADER.read_text(), flags=re.S)
    declared = sorted(set(re.findall(r"\b(?:int|size_t)\s+(lr_mmdit_\w+)\s*\(", text)))
    assert sorted(mmdit.SIGNATURES) == declared
    L = mmdit.lib()
    assert mmdit.workspace_bytes(512, 4096, 3072, 12288) > 4608 * 12288 * 2
    assert mmdit.workspace_bytes(512, 4096, 3000, 12288) == 0        # hidden not a multiple of 128
    assert mmdit.workspace_bytes(0, 0, 3072, 12288) == 0
    assert mmdit.workspace_bytes(1, 1, 3072, 12) == 0                 # mlp not a multiple of 8
    w = mmdit.Weights()
    assert L.lr_mmdit_block_bf16(None, ctypes.byref(w), None, None, 1, 1, 256, 512, None, None, None, None, 0,
                                 None) == HIP_ERROR_INVALID_VALUE
    assert L.lr_mmdit_create(None) == HIP_ERROR_INVALID_VALUE
    assert L.lr_mmdit_destroy(None) == HIP_ERROR_INVALID_VALUE
    # a workspace overlapping txt, img, the tables, t or a weight is rejected before the context is used (run in a child
    # process: a missed check would dereference the stand-in context)
    code = """
import ctypes, sys
sys.path.insert(0, %r)
from localrouter_amd import mmdit
L = mmdit.lib()
T = 1 << 40
w = mmdit.Weights(t1=T + (1 << 30), t2=T + (2 << 30), q_norm=T + (3 << 30), k_norm=T + (4 << 30),
                  txt=mmdit.StreamWeights(*[T + ((5 + i) << 30) for i in range(5)]),
                  img=mmdit.StreamWeights(*[T + ((10 + i) << 30) for i in range(5)]))
txt, img, tt, cos, sin = T + (20 << 30), T + (21 << 30), T + (22 << 30), T + (23 << 30), T + (24 << 30)
need = mmdit.workspace_bytes(16, 48, 256, 512)
ctx = ctypes.c_void_p(0x1000)
for ws in (txt + 4096, img, tt - need + 16, cos + 256, sin, w.t1, w.txt.qkv + 1024, w.img.mlp_down):
    print(L.lr_mmdit_block_bf16(ctx, ctypes.byref(w), ctypes.c_void_p(txt), ctypes.c_void_p(img), 16, 48, 256, 512,
                                ctypes.c_void_p(tt), ctypes.c_void_p(cos), ctypes.c_void_p(sin), ctypes.c_void_p(ws),
                                need, None))
""" % str(Path(__file__).resolve().parents[1])
    import subprocess
    import sys
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    assert res.stdout.split() == [str(HIP_ERROR_INVALID_VALUE)] * 8
    assert L.lr_mmdit_plan(None, 8, 16, 256, 512) == HIP_ERROR_INVALID_VALUE


def test_kmask_attention_rejects():
    L = _lib.load()
    assert L.lr_attention_kmask_workspace_bytes(0, 32) == 0
    assert L.lr_attention_kmask_workspace_bytes(218, 32) >= 2 * 218 * 32 * 128 * 2 + 218 * 4
    fake = 1 << 20   # never dereferenced: every call below is rejected before any launch
    ws = L.lr_attention_kmask_workspace_bytes(10, 2)
    args = dict(q=fake, k=fake, v=fake, out=fake, kmask=fake, n_valid=10, W=4, H=2, HK=2, nkeys=20, scale=0.088,
                q_rs=256, kv_rs=256, out_rs=256, ws=fake, ws_bytes=ws, stream=None)

    def call(**kw):
        a = dict(args, **kw)
        return L.lr_attention_kmask_bf16(*a.values())
    assert call(n_valid=0) == HIP_ERROR_INVALID_VALUE
    assert call(n_valid=21) == HIP_ERROR_INVALID_VALUE         # more kept keys than keys
    assert call(ws_bytes=ws - 1) == HIP_ERROR_INVALID_VALUE
    assert call(ws=None) == HIP_ERROR_INVALID_VALUE
    assert call(kv_rs=255) == HIP_ERROR_INVALID_VALUE
    assert call(H=3) == HIP_ERROR_INVALID_VALUE                 # H % HK
    assert call(scale=0.0) == HIP_ERROR_INVALID_VALUE
    # a workspace overlapping kmask, k, v, q or out (the compaction writes it while they are read)
    base = dict(q=1 << 40, k=2 << 40, v=3 << 40, out=4 << 40, kmask=5 << 40)
    for name in base:
        assert call(**base, ws=base[name]) == HIP_ERROR_INVALID_VALUE, name


def test_split_workspace_sizes_and_rejects():
    L = _lib.load()
    split_area = 2 * 256 * 8 * (64 * 64 * 4 + 64 * 8) + 4 * 256        # the streaming kernel's partials + counters
    assert split_area == 69207040                                        # LR_JOINT_SPLIT_BYTES
    assert L.lr_attention_ws_bytes(50220, 32, 50220, 0) == split_area   # plenty of query blocks: the split tail
    assert L.lr_attention_ws_bytes(218, 16, 50220, 1) == 0            # causal: never split
    nb = L.lr_attention_ws_bytes(218, 16, 50220, 0)                   # K6 audio-from-video: split over the keys
    assert nb >= 218 * 16 * 2 * 130 * 4 and nb != split_area
    assert L.lr_attention_ws_bytes(218, 16, 300, 0) == 0              # too few key tiles to split or stream
    assert L.lr_attention_ws_bytes(600, 16, 4096, 0) == split_area    # 48 blocks, 4,096 keys: the streaming kernel
    assert L.lr_attention_ws_bytes(600, 16, 4095, 0) == 0             # fewer keys: the pipelined kernel
    assert L.lr_attention_ws_bytes(2304, 16, 2000, 0) == 0
    fake = 1 << 20
    # a workspace overlapping q, k, v or out is rejected before any launch (the call writes partials there)
    q_, k_, v_, o_ = 1 << 40, 2 << 40, 3 << 40, 4 << 40
    rows_args = [q_, k_, v_, o_, 0, 600, 16, 16, 8000, 0, 0.088, 2048, 2048, 2048]
    nbs = L.lr_attention_ws_bytes(600, 16, 8000, 0)
    assert nbs == split_area
    for bad in (q_ + 256, k_ + (8000 - 1) * 2048 * 2, v_, o_ - nbs + 256):
        assert L.lr_attention_bf16_ws(*rows_args, bad, nbs, None) == HIP_ERROR_INVALID_VALUE, hex(bad)
    args = [fake, fake, fake, fake, 0, 218, 16, 16, 50220, 0, 0.088, 2048, 2048, 2048]
    assert L.lr_attention_bf16_ws(*args, fake, nb - 1, None) == HIP_ERROR_INVALID_VALUE   # workspace too small
    assert L.lr_attention_bf16_ws(*args, None, nb, None) == HIP_ERROR_INVALID_VALUE       # size without a pointer
    assert L.lr_attention_bf16_ws(*args, fake + 16, nb, None) == HIP_ERROR_INVALID_VALUE  # not 256-aligned


def test_image_index_is_a_permutation():
    """The key tile-image restatement the GPU layout tests decode with covers each of a tile's 8192 bf16 slots once."""
    kidx = img_index()
    assert np.array_equal(np.sort(kidx.ravel()), np.arange(8192))
    # (element units: a lane's 16 bytes are 8 elements, a 1 KB fragment 512)
    assert kidx[0, 0] == 0 and kidx[4, 0] == 8 * 8 and kidx[8, 0] == 4 * 8      # rows 4 and 8 swap lanes
    assert kidx[0, 8] == 32 * 8 and kidx[0, 16] == 512 and kidx[32, 0] == 8 * 512
