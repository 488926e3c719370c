"""The build's scratch-memory guard: the compiler's per-kernel resource remarks
are parsed, and a handoff or attention kernel that needs scratch memory fails
the build (CPU only; no compiler run)."""
from rngd_pd_amd import build

REMARKS = """\
x.hip:33:1: remark: Function Name: _ZN12_GLOBAL__N_118decode_attn_kernelILi2ELi8ELb1ELb0EEEvPKv [-Rpass-analysis=kernel-resource-usage]
   33 |     int D, uint16_t* ck) {
      | ^
x.hip:33:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]
x.hip:33:1: remark:     ScratchSize [bytes/lane]: 52 [-Rpass-analysis=kernel-resource-usage]
x.hip:33:1: remark:     VGPRs Spill: 13 [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark: Function Name: _ZN12_GLOBAL__N_111pack_kernelILb1EEEvNS_8PackArgsE [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:50:1: remark: Function Name: _ZN12_GLOBAL__N_112wgemm_kernelILi4ELi8ELi8ELb1ELb1EEEvPKt [-Rpass-analysis=kernel-resource-usage]
x.hip:50:1: remark:     ScratchSize [bytes/lane]: 640 [-Rpass-analysis=kernel-resource-usage]
"""


def test_resource_report_parses_every_kernel():
    rep = build.resource_report(REMARKS)
    assert len(rep) == 3
    attn = next(v for k, v in rep.items() if "decode_attn_kernel" in k)
    assert attn["ScratchSize [bytes/lane]"] == "52" and attn["VGPRs"] == "256"
    assert attn["VGPRs Spill"] == "13"


def test_scratch_guard_flags_only_listed_kernels():
    bad = build.scratch_kernels(build.resource_report(REMARKS))
    assert len(bad) == 1                         # the spilling GEMM is allowed, pack uses none
    assert "decode_attn_kernel" in bad[0][0] and bad[0][1] == 52


def test_build_command_asks_for_the_report():
    assert "-Rpass-analysis=kernel-resource-usage" in build.hipcc_command("/tmp/x.so")
