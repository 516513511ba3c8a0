"""The build's assembly check for VALU SGPR -> VMEM hazards (csrc/check_vmem_sgpr_hazard.py),
on hand-written gfx9 snippets: the hazard is caught straight-line and across a branch, and 5
wait states (instructions or s_nop) clear it."""
import importlib.util
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
spec = importlib.util.spec_from_file_location(
    "hz", os.path.join(ROOT, "groupgemm-cktile-optimized_amd", "csrc", "check_vmem_sgpr_hazard.py"))
hz = importlib.util.module_from_spec(spec)
spec.loader.exec_module(hz)


def _hazards(text):
    lines = text.strip().split("\n")
    _, entry = hz.scan(lines, {})
    return hz.scan(lines, entry)[0]


def test_readlane_then_dma_is_flagged():
    assert len(_hazards("""
k:
    v_readlane_b32 s4, v197, 28
    buffer_load_dwordx4 v124, s[60:63], s4 offen lds
    s_endpgm""")) == 1


def test_five_wait_states_clear_it():
    assert not _hazards("""
k:
    v_readlane_b32 s4, v197, 28
    s_nop 4
    buffer_load_dwordx4 v124, s[60:63], s4 offen lds""")
    assert not _hazards("""
k:
    v_readlane_b32 s4, v197, 28
    v_mov_b32 v1, v2
    v_mov_b32 v1, v2
    s_nop 2
    buffer_load_dwordx4 v124, s[60:63], s4 offen lds""")
    # four wait states are not enough
    assert len(_hazards("""
k:
    v_readlane_b32 s4, v197, 28
    s_nop 3
    buffer_load_dwordx4 v124, s[60:63], s4 offen lds""")) == 1


def test_rsrc_and_carry_out_and_other_registers():
    assert len(_hazards("""
k:
    v_cmp_eq_u32_e64 s[62:63], v1, v2
    buffer_store_dwordx4 v[0:3], v5, s[60:63], 0 offen""")) == 1
    assert len(_hazards("""
k:
    v_add_co_u32_e64 v1, s[8:9], v2, v3
    global_load_dword v4, v5, s[8:9]""")) == 1
    assert not _hazards("""
k:
    v_readlane_b32 s5, v197, 28
    buffer_load_dwordx4 v124, s[60:63], s4 offen lds""")


def test_hazard_across_a_branch():
    assert len(_hazards("""
k:
    v_readfirstlane_b32 s4, v1
    s_cbranch_scc1 .LBB0_2
    s_nop 7
.LBB0_2:
    buffer_load_dwordx4 v124, s[60:63], s4 offen lds""")) == 1
    # a loop back edge
    assert len(_hazards("""
k:
.LBB0_1:
    buffer_load_dwordx4 v124, s[60:63], s4 offen lds
    s_nop 7
    v_readlane_b32 s4, v197, 28
    s_cbranch_scc1 .LBB0_1
    s_endpgm""")) == 1
