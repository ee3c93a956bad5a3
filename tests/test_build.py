"""The build rejects kernels that use scratch memory (per-lane stack): parsing of
the compiler's kernel-resource-usage remarks."""

from aster_amd import build


def test_scratch_kernels_are_reported():
    remarks = "\n".join([
        "x.hip:1:1: remark: Function Name: kern_a [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark: Function Name: kern_b [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     ScratchSize [bytes/lane]: 544 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert build._scratch_kernels(remarks) == ["kern_b (544 bytes/lane)"]
    assert build._scratch_kernels("") == []


def test_build_flags_request_resource_remarks():
    assert build.RESOURCE_REMARKS == "-Rpass-analysis=kernel-resource-usage"
    assert "-packed-fp32-ops" in build.FLAGS
