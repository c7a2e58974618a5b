"""The MFMA-result hazard scan (torchnative_amd/hazard_scan.py): pinned on
planted assembly, then run over the library's own gfx950 assembly, which
must have no early read."""

import shutil

import pytest

from torchnative_amd import hazard_scan as H

MFMA = "v_mfma_f32_32x32x16_bf16 v[0:15], v[20:23], v[24:27], v[0:15]"


def _fn(*body):
    return "\n".join(["_Z4testv:", *body, "s_endpgm"])


def test_a_read_right_after_the_product_is_found():
    found = H.scan_text(_fn(MFMA, "v_max_f32 v40, v3, v4"))
    assert len(found) == 1 and found[0][3] == 0


def test_a_read_behind_a_branch_is_found():
    """The case the compiler once got wrong: the read sits in the branch target."""
    asm = _fn(MFMA, "s_cbranch_scc1 .LBB0_2", "s_nop 7", "s_nop 7", "s_nop 3", ".LBB0_2:", "v_max_f32 v40, v7, v4")
    found = H.scan_text(asm)
    assert len(found) == 1 and "v_max_f32" in found[0][2] and found[0][3] == 1


def test_a_path_with_no_active_lane_reads_nothing_until_exec_is_set():
    # the fall-through of s_cbranch_execnz runs with exec == 0: no read there ...
    asm = _fn(MFMA, "s_cbranch_execnz .LBB0_2", "v_max_f32 v40, v3, v4", ".LBB0_2:", "s_nop 7", "s_nop 7", "s_nop 3",
              "v_add_f32 v9, v1, v2")
    assert H.scan_text(asm) == []
    # ... until exec is written again
    asm = _fn(MFMA, "s_cbranch_execnz .LBB0_2", "s_mov_b64 exec, -1", "v_max_f32 v40, v3, v4", ".LBB0_2:",
              "s_nop 7", "s_nop 7", "s_nop 3")
    assert len(H.scan_text(asm)) == 1
    # the taken branch of s_cbranch_execz likewise
    asm = _fn(MFMA, "s_cbranch_execz .LBB0_2", "s_nop 7", "s_nop 7", "s_nop 3", "s_endpgm", ".LBB0_2:",
              "v_max_f32 v40, v3, v4")
    assert H.scan_text(asm) == []


def test_enough_wait_states_and_accumulation_are_not_hazards():
    assert H.scan_text(_fn(MFMA, "s_nop 7", "s_nop 7", "s_nop 1", "v_max_f32 v40, v3, v4")) == []
    # another product accumulating into the same registers (srcC) is not a read
    assert H.scan_text(_fn(MFMA, MFMA, "s_nop 7", "s_nop 7", "s_nop 1", "v_add_f32 v40, v0, v1")) == []
    # 17 wait states are one short
    assert len(H.scan_text(_fn(MFMA, "s_nop 7", "s_nop 7", "s_nop 0", "v_max_f32 v40, v3, v4"))) == 1
    # a 16x16 product needs 8
    m16 = "v_mfma_f32_16x16x32_bf16 v[0:3], v[20:23], v[24:27], v[0:3]"
    assert H.scan_text(_fn(m16, "s_nop 7", "v_add_f32 v9, v1, v2")) == []
    assert len(H.scan_text(_fn(m16, "s_nop 6", "v_add_f32 v9, v1, v2"))) == 1


@pytest.mark.skipif(shutil.which(H.build.HIPCC) is None and not __import__("os").path.exists(H.build.HIPCC),
                    reason="hipcc is not installed")
def test_the_librarys_assembly_reads_no_mfma_result_early():
    results = H.scan_sources()
    bad = [(src, f) for src, found in results.items() for f in found]
    assert not bad, "\n".join(f"{src}: {f[0][:60]}: {f[2]} after {f[3]} wait states" for src, f in bad[:20])
