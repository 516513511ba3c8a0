"""The build's assembly checks, on hand-written gfx9 snippets.

- VALU SGPR -> VMEM hazards (csrc/check_vmem_sgpr_hazard.py): caught straight-line and across a
  branch; 5 wait states (instructions or s_nop) clear them.
- Accumulator reads after an inline-asm MFMA (csrc/check_mfma_acc_hazard.py): caught within 19
  wait states, across a fall-through and a loop's back edge; reads of other AGPRs pass; SGPR
  spill traffic in a K-loop block (many MFMAs) fails, in a single step's block it does not.
- The product library carries no cycle stamps (those are the `make stamps` build's).
- Every GEMM instance of the product library compiles with 0 VGPR spills and 0 scratch (the
  compiler's resource report, lib/resource_usage.txt).
"""
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


# ---- accumulator reads after an inline-asm MFMA (csrc/check_mfma_acc_hazard.py) ----
spec2 = importlib.util.spec_from_file_location(
    "acc", os.path.join(ROOT, "groupgemm-cktile-optimized_amd", "csrc", "check_mfma_acc_hazard.py"))
acc = importlib.util.module_from_spec(spec2)
spec2.loader.exec_module(acc)


def _acc(body):
    return acc.scan_text("\n_Zk:\n" + body.strip() + "\n.Lfunc_end0:\n")


def test_accumulator_read_right_after_mfma_is_flagged():
    bad, _ = _acc("""
    v_mfma_f32_16x16x32_bf16 a[4:7], v[0:3], v[8:11], a[4:7]
    v_accvgpr_read_b32 v20, a5""")
    assert len(bad) == 1 and "after 0 wait states" in bad[0]


def test_nineteen_wait_states_or_other_registers_clear_it():
    bad, _ = _acc("""
    v_mfma_f32_16x16x32_bf16 a[4:7], v[0:3], v[8:11], a[4:7]
    s_nop 7
    s_nop 7
    s_nop 2
    v_accvgpr_read_b32 v20, a5""")
    assert not bad
    bad, _ = _acc("""
    v_mfma_f32_16x16x32_bf16 a[4:7], v[0:3], v[8:11], a[4:7]
    s_nop 7
    s_nop 7
    s_nop 1
    v_accvgpr_read_b32 v20, a5""")
    assert len(bad) == 1  # 18 wait states
    bad, _ = _acc("""
    v_mfma_f32_16x16x32_bf16 a[4:7], v[0:3], v[8:11], a[4:7]
    v_accvgpr_read_b32 v20, a8
    global_store_dwordx4 v[0:1], a[0:3], off""")
    assert not bad


def test_store_of_an_mfma_result_and_a_read_across_a_branch_are_flagged():
    bad, _ = _acc("""
    v_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[8:11], a[0:3]
    global_store_dwordx4 v[4:5], a[0:3], off""")
    assert len(bad) == 1
    # through a back edge: the MFMA ends the loop block, the read starts it
    bad, _ = _acc("""
.LBB0_1:
    v_accvgpr_read_b32 v20, a2
    v_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[8:11], a[0:3]
    s_cbranch_scc1 .LBB0_1
    s_endpgm""")
    assert len(bad) == 1
    # through a fall-through into the next block
    bad, _ = _acc("""
    v_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[8:11], a[0:3]
.LBB0_2:
    v_accvgpr_read_b32 v20, a1""")
    assert len(bad) == 1


def test_spill_traffic_in_the_k_loop_is_flagged():
    mfma = "    v_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[8:11], a[0:3]"
    _, spills = _acc(".LBB0_3:\n    v_readlane_b32 s4, v185, 12\n" + "\n".join([mfma] * acc.LOOP_MFMAS))
    assert len(spills) == 1
    _, spills = _acc(".LBB0_3:\n    v_readlane_b32 s4, v185, 12\n" + "\n".join([mfma] * 16))
    assert not spills  # a single step's block (first or checked steps) may reload


def test_product_library_has_no_cycle_stamps():
    """The cycle stamps (GG_STAMPS) are compiled only into lib_stamps/ (`make stamps`): the product
    library exports none of their read-back functions."""
    import ctypes
    import pytest
    path = os.path.join(ROOT, "groupgemm-cktile-optimized_amd", "lib", "libgg_mi355x.so")
    if not os.path.exists(path):
        pytest.skip("library not built")
    lib = ctypes.CDLL(path)
    assert not hasattr(lib, "gg_stamps_read_p0") and not hasattr(lib, "gg_stamps_clear_p18")


def test_no_vgpr_spills_or_scratch_in_any_instance():
    """The compiler's report of every grouped_gemm_kernel instance (Function Name, then its
    VGPRs Spill and ScratchSize lines) shows no VGPR spill and no scratch: spilled values would
    travel through memory, next to the operand DMAs."""
    import re
    import pytest
    path = os.path.join(ROOT, "groupgemm-cktile-optimized_amd", "lib", "resource_usage.txt")
    if not os.path.exists(path):
        pytest.skip("library not built")
    seen, bad, cur = 0, [], None
    with open(path, errors="replace") as f:
        for line in f:
            m = re.search(r"Function Name: (\S+)", line)
            if m:
                cur = m.group(1) if "grouped_gemm_kernel" in m.group(1) else None
                seen += cur is not None
                continue
            if cur is None:
                continue
            m = re.search(r"\s(VGPRs Spill|ScratchSize \[bytes/lane\]): (\d+)", line)
            if m and int(m.group(2)) != 0:
                bad.append((cur, m.group(1), int(m.group(2))))
    assert seen >= 60, seen  # every (type, mode, shape, variant) instance is in the report
    assert not bad, bad
