"""The build's guard on the DMA-staged forward kernels (``_build.check_dma_spills``).

Those kernels wait for their tile loads with a fixed ``s_waitcnt vmcnt(4)`` that counts
only the loads their loop issues; a VGPR spill (a scratch access) between a DMA and its
wait would release the wait early.  The guard reads the compiler's per-kernel resource
remarks and fails the build when such a kernel spills.  These tests feed it remark text
with a planted spilling variant."""

from __future__ import annotations

import pytest

from kohakutt_amd import _build

BF16_DMA_32 = "_ZN3kmi3fwd15attn_fwd_kernelIDF16bLi64ELi2ELi0ELb0ELi32ELi4EEEvNS0_10AttnParamsE"
F16_DMA_64 = "_ZN3kmi3fwd15attn_fwd_kernelIDF16_Li64ELi4ELi0ELb0ELi32ELi4EEEvNS0_10AttnParamsE"
ROWSPLIT_64 = "_ZN3kmi3fwd15attn_fwd_kernelIDF16bLi64ELi4ELi0ELb1ELi32ELi4EEEvNS0_10AttnParamsE"
MASKED_32 = "_ZN3kmi3fwd15attn_fwd_kernelIDF16bLi64ELi2ELi2ELb0ELi32ELi4EEEvNS0_10AttnParamsE"
D128 = "_ZN3kmi3fwd15attn_fwd_kernelIDF16bLi128ELi2ELi0ELb0ELi32ELi4EEEvNS0_10AttnParamsE"
DECODE = "_ZN3kmi3fwd18attn_decode_kernelIDF16bLi64ELi0EEEvNS0_10AttnParamsE"


def _remarks(*kernels):
    """Remark text in the compiler's format for (name, vgpr_spill, scratch) triples."""
    lines = []
    for name, spill, scratch in kernels:
        at = "attention_kernels.hpp:1184:1: remark: "
        lines += [
            f"{at}Function Name: {name} [-Rpass-analysis=kernel-resource-usage]",
            f"{at}    VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]",
            f"{at}    ScratchSize [bytes/lane]: {scratch} [-Rpass-analysis=kernel-resource-usage]",
            f"{at}    SGPRs Spill: 139 [-Rpass-analysis=kernel-resource-usage]",
            f"{at}    VGPRs Spill: {spill} [-Rpass-analysis=kernel-resource-usage]",
        ]
    return "\n".join(lines)


def test_which_instantiations_are_dma_staged():
    assert _build.is_dma_forward(BF16_DMA_32)
    assert _build.is_dma_forward(F16_DMA_64)
    for name in (ROWSPLIT_64, MASKED_32, D128, DECODE):
        assert not _build.is_dma_forward(name), name


def test_clean_build_passes_and_counts_the_dma_kernels():
    text = _remarks((BF16_DMA_32, 0, 0), (F16_DMA_64, 0, 0), (MASKED_32, 7, 16), (DECODE, 0, 0))
    assert _build.check_dma_spills(text) == 2


@pytest.mark.parametrize("spill,scratch", [(3, 12), (0, 8)])
def test_planted_spilling_dma_variant_fails_the_build(spill, scratch):
    text = _remarks((MASKED_32, 0, 0), (BF16_DMA_32, spill, scratch), (F16_DMA_64, 0, 0))
    with pytest.raises(RuntimeError, match="attn_fwd_kernelIDF16bLi64ELi2ELi0"):
        _build.check_dma_spills(text)


def test_the_guarded_unit_is_compiled_with_resource_remarks():
    assert _build.RESOURCE_REMARKS in _build.SOURCE_FLAGS["attention_d64.hip"]
