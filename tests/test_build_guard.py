"""The build's guard for kernels that issue loads from inline asm: it reads
the compiler's resource-usage remarks and fails on scratch use, spills or a
VGPR count past the kernel's budget (synthetic remark text, no compiler)."""

from pathlib import Path

import pytest

import build_lib

_OK = """x.hip:549:1: remark: Function Name: _ZN12_GLOBAL__N_124project_cols_pipe_kernelILi2ELi128ELi16ELi4EEEv [-Rpass]
x.hip:549:1: remark:     TotalSGPRs: 44 [-Rpass]
x.hip:549:1: remark:     VGPRs: 244 [-Rpass]
x.hip:549:1: remark:     AGPRs: 0 [-Rpass]
x.hip:549:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass]
x.hip:549:1: remark:     Occupancy [waves/SIMD]: 2 [-Rpass]
x.hip:549:1: remark:     SGPRs Spill: 0 [-Rpass]
x.hip:549:1: remark:     VGPRs Spill: 0 [-Rpass]
x.hip:120:1: remark: Function Name: _ZN12_GLOBAL__N_121project_direct_kernelILi2ELi128ELi4EEEv [-Rpass]
x.hip:120:1: remark:     VGPRs: 300 [-Rpass]
x.hip:120:1: remark:     ScratchSize [bytes/lane]: 64 [-Rpass]
"""
SRC = Path("tm_project.hip")


def test_guard_accepts_clean_kernel_and_ignores_others():
    build_lib._check_asm_load_kernels(SRC, _OK)  # project_direct_kernel is not an asm-load kernel


@pytest.mark.parametrize("old,new", [("VGPRs: 244", "VGPRs: 260"), ("VGPRs Spill: 0", "VGPRs Spill: 3"),
                                     ("ScratchSize [bytes/lane]: 0", "ScratchSize [bytes/lane]: 16"),
                                     ("SGPRs Spill: 0", "SGPRs Spill: 1")])
def test_guard_rejects_spill_scratch_or_budget(old, new):
    with pytest.raises(RuntimeError, match="project_cols_pipe_kernel"):
        build_lib._check_asm_load_kernels(SRC, _OK.replace(old, new, 1))


def test_guard_requires_the_remarks():
    with pytest.raises(RuntimeError, match="no resource remarks"):
        build_lib._check_asm_load_kernels(SRC, "")
