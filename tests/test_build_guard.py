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
