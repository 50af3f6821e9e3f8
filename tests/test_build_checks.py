"""The build's register check: a kernel that spills VGPRs, uses scratch
memory or holds more static LDS than its family declares (a register array
the compiler moved into LDS) fails the build
(mxflashattn_amd._build.check_resource_usage), read from hipcc's
kernel-resource-usage remarks."""

from __future__ import annotations

import pytest

from mxflashattn_amd import _build


def remarks(name: str, spill: int, scratch: int, lds: int = 0) -> str:
    loc = "split_kernels.h:1:1: remark:"
    return "\n".join([
        f"{loc} Function Name: {name} [-Rpass-analysis=kernel-resource-usage]",
        f"{loc}     TotalSGPRs: 80 [-Rpass-analysis=kernel-resource-usage]",
        f"{loc}     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]",
        f"{loc}     AGPRs: 0 [-Rpass-analysis=kernel-resource-usage]",
        f"{loc}     ScratchSize [bytes/lane]: {scratch} [-Rpass-analysis=kernel-resource-usage]",
        f"{loc}     Occupancy [waves/SIMD]: 2 [-Rpass-analysis=kernel-resource-usage]",
        f"{loc}     SGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]",
        f"{loc}     VGPRs Spill: {spill} [-Rpass-analysis=kernel-resource-usage]",
        f"{loc}     LDS Size [bytes/block]: {lds} [-Rpass-analysis=kernel-resource-usage]",
    ]) + "\n"


def test_clean_kernels_pass():
    text = remarks("_Z1av", 0, 0) + remarks("_Z1bv", 0, 0)
    kernels = _build.check_resource_usage("unit.hip", text)
    assert set(kernels) == {"_Z1av", "_Z1bv"}
    assert kernels["_Z1av"]["VGPRs"] == "256"


@pytest.mark.parametrize("spill,scratch", [(105, 280), (0, 32)])
def test_spills_or_scratch_fail_the_build(spill, scratch):
    text = remarks("_Z1av", 0, 0) + remarks("_Z8spillingv", spill, scratch)
    with pytest.raises(RuntimeError, match="_Z8spillingv"):
        _build.check_resource_usage("unit.hip", text)


def test_compile_command_asks_for_the_remarks():
    cmd = _build.compile_command(_build.CSRC_DIR / "split_hd64.hip", _build.LIB_DIR / "x.o")
    assert _build.RESOURCE_REMARKS in cmd


PARTIAL = "_ZN4mxfa20split_partial_kernelILi64ELi2ENS_4BF16EEEvPKiiNS_12DecodeParamsE"
COMBINE = "_ZN4mxfa20split_combine_kernelILi64ENS_4BF16EEEvPKiPKfS4_iiiiiiiNS_13CombineParamsE"


def test_declared_static_lds_passes():
    text = remarks(PARTIAL, 0, 0, lds=32) + remarks(COMBINE, 0, 0, lds=6144)
    assert set(_build.check_resource_usage("unit.hip", text)) == {PARTIAL, COMBINE}


@pytest.mark.parametrize("name,lds", [(PARTIAL, 9216), (COMBINE, 6144 + 36 * 256)])
def test_arrays_promoted_to_lds_fail_the_build(name, lds):
    # 9216 bytes: nine ints per thread of a 256-thread workgroup, what a
    # per-lane array of the split kernel took once the compiler moved it
    # from registers into LDS.
    with pytest.raises(RuntimeError, match="static LDS"):
        _build.check_resource_usage("unit.hip", remarks(name, 0, 0, lds=lds))
