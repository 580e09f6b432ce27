"""The build recipe refuses kernels that use scratch memory (register spills or
private arrays), which cost the GEMMs up to 10x without any other symptom."""
from __future__ import annotations

from cleave_amd.build import scratch_users


def test_scratch_report_parser_flags_only_nonzero_kernels():
    report = "\n".join([
        "a.hip:1:1: remark: Function Name: kern_clean [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:1:1: remark:     VGPRs: 64 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark: Function Name: kern_spills [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark:     ScratchSize [bytes/lane]: 484 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert scratch_users(report) == ["kern_spills: 484 bytes/lane"]
    assert scratch_users("no remarks at all") == []
