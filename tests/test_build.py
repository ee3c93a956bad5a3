"""The build rejects kernels that spill registers: per-lane scratch (stack) memory, or
AGPRs used as spill space (every MFMA accumulator is meant to live in VGPRs), outside
the exact fp32 VALU decode kernels known to spill that way: parsing of the compiler's
kernel-resource-usage remarks."""

from aster_amd import build


def _remark(line, text):
    return f"x.hip:{line}:1: remark: {text} [-Rpass-analysis=kernel-resource-usage]"


def test_register_spills_are_reported():
    remarks = "\n".join([
        _remark(1, "Function Name: kern_a"),
        _remark(1, "    AGPRs: 0"),
        _remark(1, "    ScratchSize [bytes/lane]: 0"),
        _remark(9, "Function Name: kern_b"),
        _remark(9, "    VGPRs: 256"),
        _remark(9, "    AGPRs: 0"),
        _remark(9, "    ScratchSize [bytes/lane]: 544"),
        _remark(20, "Function Name: kern_c"),
        _remark(20, "    VGPRs: 256"),
        _remark(20, "    AGPRs: 41"),
        _remark(20, "    ScratchSize [bytes/lane]: 0"),
        _remark(30, "Function Name: _ZN4astr4attn12_GLOBAL__N_118decode_valu_kernelIfLi128ELi4ELi4EEEvNS0_8AttnArgsE"),
        _remark(30, "    AGPRs: 40"),
        _remark(30, "    ScratchSize [bytes/lane]: 0"),
    ])
    assert build._scratch_kernels(remarks) == ["kern_b (544 bytes/lane of scratch)",
                                               "kern_c (41 AGPRs: VGPRs spilled)"]
    assert build._scratch_kernels("") == []


def test_build_flags_request_resource_remarks():
    assert build.RESOURCE_REMARKS == "-Rpass-analysis=kernel-resource-usage"
    assert "-packed-fp32-ops" in build.FLAGS
