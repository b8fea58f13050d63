"""The build's scratch guard (localrouter_amd/build.py): the compiler's kernel-resource-usage remarks are parsed, and a
kernel with more scratch than its budget fails the build. The streaming and INT8 attention kernels count their
direct-to-LDS refills with explicit vmcnt waits, which a spill among those loads would break without a compile error."""
from __future__ import annotations

import json

from localrouter_amd import build

SAMPLE = """\
/src/attn_stream.hip:181:1: remark: Function Name: _ZN2lr12_GLOBAL__N_118attn_stream_kernelENS_8AttnArgsE [-Rpass-analysis=kernel-resource-usage]
  181 | __global__ void attn_stream_kernel(AttnArgs a) {
      | ^
/src/attn_stream.hip:181:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]
/src/attn_stream.hip:181:1: remark:     AGPRs: 128 [-Rpass-analysis=kernel-resource-usage]
/src/attn_stream.hip:181:1: remark:     ScratchSize [bytes/lane]: 8 [-Rpass-analysis=kernel-resource-usage]
/src/attn_stream.hip:181:1: remark:     Occupancy [waves/SIMD]: 2 [-Rpass-analysis=kernel-resource-usage]
/src/mmdit.hip:44:1: remark: Function Name: _ZN2lr12_GLOBAL__N_111silu_kernelEPKtPti [-Rpass-analysis=kernel-resource-usage]
/src/mmdit.hip:44:1: remark:     VGPRs: 6 [-Rpass-analysis=kernel-resource-usage]
/src/mmdit.hip:44:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
"""


def test_remarks_are_parsed():
    r = build.kernel_resources(SAMPLE)
    k = "_ZN2lr12_GLOBAL__N_118attn_stream_kernelENS_8AttnArgsE"
    assert r[k] == {"VGPRs": 128, "AGPRs": 128, "ScratchSize": 8, "Occupancy": 2}
    assert r["_ZN2lr12_GLOBAL__N_111silu_kernelEPKtPti"]["ScratchSize"] == 0


def test_budget_flags_a_spill():
    ok = build.kernel_resources(SAMPLE)
    assert build.scratch_violations(ok) == []
    # planted: the streaming kernel spilling more, and a kernel with no budget spilling at all
    bad = {"_ZN2lr12_GLOBAL__N_118attn_stream_kernelENS_8AttnArgsE": {"ScratchSize": 16},
           "_ZN2lr12_GLOBAL__N_111silu_kernelEPKtPti": {"ScratchSize": 4},
           "_ZN2lr2i812_GLOBAL__N_114i8_attn_kernelILi128ELi4ELi128EEEvNS0_8AttnArgsE": {"ScratchSize": 8}}
    v = build.scratch_violations(bad)
    assert len(v) == 2 and any("attn_stream_kernel" in x for x in v) and any("silu_kernel" in x for x in v)


def test_built_library_is_within_budget():
    """The report of the last build (written next to the objects): every kernel within its budget, the two
    streaming kernels present."""
    if not build.RESOURCES.exists():
        import pytest
        pytest.skip("no build report (build() writes it)")
    res = json.loads(build.RESOURCES.read_text())
    assert build.scratch_violations(res) == []
    assert any("attn_stream_kernel" in k for k in res) and any("i8_attn_kernel" in k for k in res)
    stream = next(v for k, v in res.items() if "attn_stream_kernel" in k)
    assert stream["VGPRs"] + stream["AGPRs"] <= 256 and stream["Occupancy"] == 2


ASM = """\
_ZN2lr12_GLOBAL__N_118attn_stream_kernelENS_8AttnArgsE: ; @_ZN2lr12_GLOBAL__N_118attn_stream_kernelENS_8AttnArgsE
; %bb.0:
	s_load_dwordx2 s[0:1], s[0:1], 0x0
	scratch_store_dword off, v6, off        ; 4-byte Folded Spill
.LBB0_168:                              ; =>This Loop Header: Depth=1
	v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]
.LBB0_172:                              ;   in Loop: Header=BB0_168 Depth=1
	s_barrier
	s_cbranch_scc1 .LBB0_168
; %bb.407:
	scratch_load_dword v0, off, off         ; 4-byte Folded Reload
	s_endpgm
.Lfunc_end0:
"""


def test_loop_scan_finds_a_spill_inside_the_loop():
    """The assembly scan (build.loop_scratch_ops): the present spill, stored before the loop and reloaded after it,
    passes; the same store planted in a loop block (header or body) is reported."""
    k = "attn_stream_kernel"
    assert build.loop_scratch_ops(ASM, k) == (2, [])
    planted = ASM.replace("\ts_barrier\n", "\ts_barrier\n\tscratch_store_dword off, v9, off offset:4\n")
    total, inside = build.loop_scratch_ops(planted, k)
    assert total == 3 and len(inside) == 1 and "v9" in inside[0]
    planted = ASM.replace("\tv_mfma_f32", "\tscratch_load_dword v1, off, off\n\tv_mfma_f32")
    assert len(build.loop_scratch_ops(planted, k)[1]) == 1


def test_built_kernels_keep_scratch_out_of_their_loops():
    """The last build's generated assembly of the two kernels with a scratch budget: no scratch access in a loop."""
    import re
    import pytest
    for src, kernel in build.LOOP_SCAN:
        path = build.PKG / "_build" / src.replace(".hip", ".s")
        if not path.exists():
            pytest.skip("no generated assembly (build() writes it)")
        asm = path.read_text()
        names = set(re.findall(r"^(_Z\S*" + re.escape(kernel) + r"\S*):", asm, re.M))
        assert names
        for name in names:
            assert build.loop_scratch_ops(asm, name)[1] == [], name
