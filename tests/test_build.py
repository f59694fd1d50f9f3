"""The build's reading of the compiler's resource remarks (CPU): vector-register spills per kernel, and the names
of the benchmarked kernels it watches."""
from nvs_amd import build as nb

REMARKS = """\
spec_sampler.hip:1696:1: remark: Function Name: _ZN12_GLOBAL__N_118markov_draw_kernelILi1ELb1ELb1EEEvNS_15MarkovSplitArgsE [-Rpass-analysis=kernel-resource-usage]
spec_sampler.hip:1696:1: remark:     TotalSGPRs: 106 [-Rpass-analysis=kernel-resource-usage]
spec_sampler.hip:1696:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]
spec_sampler.hip:1696:1: remark:     ScratchSize [bytes/lane]: 32 [-Rpass-analysis=kernel-resource-usage]
spec_sampler.hip:1696:1: remark:     SGPRs Spill: 121 [-Rpass-analysis=kernel-resource-usage]
spec_sampler.hip:1696:1: remark:     VGPRs Spill: 5 [-Rpass-analysis=kernel-resource-usage]
spec_sampler.hip:2047:1: remark: Function Name: _ZN12_GLOBAL__N_113select_kernelILi0ELi0ELb1ELb0EEEvNS_7SelArgsE [-Rpass-analysis=kernel-resource-usage]
spec_sampler.hip:2047:1: remark:     ScratchSize [bytes/lane]: 36 [-Rpass-analysis=kernel-resource-usage]
spec_sampler.hip:2047:1: remark:     SGPRs Spill: 24 [-Rpass-analysis=kernel-resource-usage]
spec_sampler.hip:2047:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
"""


def test_vgpr_spills_are_read_per_kernel():
    spills = nb._vgpr_spills_by_kernel(REMARKS.splitlines())
    assert spills == {
        "_ZN12_GLOBAL__N_118markov_draw_kernelILi1ELb1ELb1EEEvNS_15MarkovSplitArgsE": 5,
        # private memory without spilled vector registers (a private array) is not a spill
        "_ZN12_GLOBAL__N_113select_kernelILi0ELi0ELb1ELb0EEEvNS_7SelArgsE": 0,
    }


def test_watched_names_match_the_benchmarked_instantiations():
    names = [
        "_ZN12_GLOBAL__N_117attn_split_kernelILi1EEEvNS_8AttnArgsE",
        "_ZN12_GLOBAL__N_113select_kernelILi0ELi0ELb1ELb0EEEvNS_7SelArgsE",
        "_ZN12_GLOBAL__N_113select_kernelILi1ELi0ELb1ELb0EEEvNS_7SelArgsE",
        "_ZN12_GLOBAL__N_118markov_draw_kernelILi1ELb1ELb1EEEvNS_15MarkovSplitArgsE",
        "_ZN12_GLOBAL__N_125qk_norm_rope_store_kernelILi1EEEvNS_12NormRopeArgsE",
    ]
    for pattern in nb.HOT_KERNELS:
        assert sum(pattern in n for n in names) == 1, pattern
    # other instantiations are not watched
    assert not any(p in "_ZN12_GLOBAL__N_113select_kernelILi0ELi0ELb0ELb1EEEvNS_7SelArgsE" for p in nb.HOT_KERNELS)


def test_remark_source_excerpts_are_not_shown():
    assert nb._is_remark_context(" 1696 | __global__ __launch_bounds__(kSelThreads, 4) void markov_draw_kernel(")
    assert nb._is_remark_context("      | ^")
    assert not nb._is_remark_context("spec_sampler.hip:12:3: warning: unused variable 'x'")
