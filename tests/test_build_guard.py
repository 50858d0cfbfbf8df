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
                                     ("ScratchSize [bytes/lane]: 0", "ScratchSize [bytes/lane]: 16")])
def test_guard_rejects_spill_scratch_or_budget(old, new):
    with pytest.raises(RuntimeError, match="project_cols_pipe_kernel"):
        build_lib._check_asm_load_kernels(SRC, _OK.replace(old, new, 1))


def test_guard_accepts_sgpr_spills_to_vgpr_lanes():
    build_lib._check_asm_load_kernels(SRC, _OK.replace("SGPRs Spill: 0", "SGPRs Spill: 4", 1))


def test_guard_requires_the_remarks():
    with pytest.raises(RuntimeError, match="no resource remarks"):
        build_lib._check_asm_load_kernels(SRC, "")


def _fn(body: str) -> str:
    return "_Z4kernv:\n" + body + "\n.Lfunc_end0:\n"


def test_isa_check_accepts_waited_load():
    import isa_check

    asm = _fn("""\tglobal_load_dwordx4 v[4:7], v[0:1], off
\tglobal_load_dwordx4 v[8:11], v[0:1], off offset:16
\ts_waitcnt vmcnt(1)
\tv_add_f32_e32 v12, v4, v5
\ts_waitcnt vmcnt(0)
\tv_add_f32_e32 v13, v8, v9
\ts_endpgm""")
    assert isa_check.check_function(asm, "_Z4kernv") == []


def test_isa_check_flags_early_read_and_reuse():
    import isa_check

    asm = _fn("""\tglobal_load_dwordx4 v[4:7], v[0:1], off
\tglobal_load_dwordx4 v[8:11], v[0:1], off offset:16
\ts_waitcnt vmcnt(1)
\tv_add_f32_e32 v12, v8, v5
\tv_mov_b32_e32 v9, 0
\ts_endpgm""")
    kinds = [k for _, k, _ in isa_check.check_function(asm, "_Z4kernv")]
    assert kinds == ["read", "overwrite"]


def test_isa_check_follows_branches():
    """A wait on one path only: the join keeps the load pending."""
    import isa_check

    asm = _fn("""\tglobal_load_dword v4, v[0:1], off
\ts_cbranch_scc1 .LBB0_2
\ts_waitcnt vmcnt(0)
.LBB0_2:
\tv_add_f32_e32 v5, v4, v4
\ts_endpgm""")
    assert [k for _, k, _ in isa_check.check_function(asm, "_Z4kernv")] == ["read"]
