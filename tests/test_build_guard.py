"""The build's guard for the kernels' untracked LDS reads: hipcc's
kernel-resource-usage remarks are parsed per kernel and any kernel with private
scratch or spilled vector registers fails the build (a spill of an inline-asm
LDS read's destination before its explicit wait would store stale data); scalar
registers spilled into VGPR lanes without scratch pass."""

from specfold_amd.build import kernel_resources, spilling_kernels

SAMPLE = """\
x.hip:10:1: remark: Function Name: _Z5cleanv [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     VGPRs: 100 [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     SGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark: Function Name: _Z6spillsv [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark:     ScratchSize [bytes/lane]: 16 [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark:     SGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark:     VGPRs Spill: 4 [-Rpass-analysis=kernel-resource-usage]
x.hip:30:1: remark: Function Name: _Z7scratchv [-Rpass-analysis=kernel-resource-usage]
x.hip:30:1: remark:     ScratchSize [bytes/lane]: 32 [-Rpass-analysis=kernel-resource-usage]
x.hip:30:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark: Function Name: _Z5lanesv [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark:     VGPRs: 158 [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark:     SGPRs Spill: 4 [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:50:1: remark: Function Name: _Z10sgprscratchv [-Rpass-analysis=kernel-resource-usage]
x.hip:50:1: remark:     ScratchSize [bytes/lane]: 8 [-Rpass-analysis=kernel-resource-usage]
x.hip:50:1: remark:     SGPRs Spill: 40 [-Rpass-analysis=kernel-resource-usage]
x.hip:50:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
"""


def test_parser_flags_spills_and_scratch():
    res = kernel_resources(SAMPLE)
    assert set(res) == {"_Z5cleanv", "_Z6spillsv", "_Z7scratchv", "_Z5lanesv", "_Z10sgprscratchv"}
    assert res["_Z6spillsv"]["VGPRs Spill"] == "4"
    bad = spilling_kernels(res)
    # VGPR spills and any scratch fail; SGPRs spilled to VGPR lanes (no scratch) pass
    assert len(bad) == 3 and bad[0].startswith("_Z6spillsv") and bad[1].startswith("_Z7scratchv")
    assert bad[2].startswith("_Z10sgprscratchv")
    assert spilling_kernels({"_Z5cleanv": res["_Z5cleanv"]}) == []
