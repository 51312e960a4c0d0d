"""The build's scratch guard: kernels that must not spill (the MLA decode,
whose inline-assembly waits and hazard cover assume its spill-free register
allocation) are found in the compiler's resource remarks."""

from __future__ import annotations

from flydsl_amd import build

REMARKS = """\
x/mla_fp8.hip:468:1: remark: Function Name: _ZN12_GLOBAL__N_121mla_fp8_decode_kernelILb1ELi1EEEv18pa_mla_decode_args [-Rpass-analysis=kernel-resource-usage]
x/mla_fp8.hip:468:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]
x/mla_fp8.hip:468:1: remark:     ScratchSize [bytes/lane]: 84 [-Rpass-analysis=kernel-resource-usage]
x/mla_fp8.hip:468:1: remark: Function Name: _ZN12_GLOBAL__N_121mla_fp8_decode_kernelILb0ELi1EEEv18pa_mla_decode_args [-Rpass-analysis=kernel-resource-usage]
x/mla_fp8.hip:468:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x/mla_fp8.hip:700:1: remark: Function Name: _ZN12_GLOBAL__N_121mla_fp8_reduce_kernelE18pa_mla_reduce_args [-Rpass-analysis=kernel-resource-usage]
x/mla_fp8.hip:700:1: remark:     ScratchSize [bytes/lane]: 16 [-Rpass-analysis=kernel-resource-usage]
"""


def test_scratch_users_names_only_the_guarded_kernels_that_spill():
    got = build.scratch_users(REMARKS, ("mla_fp8_decode_kernel",))
    assert got == [("_ZN12_GLOBAL__N_121mla_fp8_decode_kernelILb1ELi1EEEv18pa_mla_decode_args", 84)]
    assert build.scratch_users(REMARKS, ()) == []


def test_guarded_sources_are_compiled_with_resource_remarks():
    cmd = build._compile_cmd("/x/mla_fp8.hip", "/x/o.o")
    assert "-Rpass-analysis=kernel-resource-usage" in cmd
    assert "-Rpass-analysis=kernel-resource-usage" not in build._compile_cmd("/x/pa_fp8.hip", "/x/o.o")
    assert "-DPA_FP8_CHECKED" in build._compile_cmd("/x/pa_fp8.hip", "/x/o.o", ("PA_FP8_CHECKED",))
