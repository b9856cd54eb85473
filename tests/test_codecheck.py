"""The machine-code check of the built library (duck_gym_amd/codecheck.py):
no vector instruction placed where the exec mask is zero, i.e. between a
divergent loop's exit (`s_cbranch_execnz` falling through) and the next
write of exec.  Pinned on hand-written disassembly first, then applied to
the built libduck_hip.so."""

from pathlib import Path

import pytest

from duck_gym_amd import codecheck as C

HEAD = "0000000000001000 <kernel>:\n"


def _asm(lines):
    out, address = [HEAD], 0x1000
    for text in lines:
        out.append(f"\t{text:58s} // {address:012X}: 00000000\n")
        address += 4
    return "".join(out)


LOOP = ["s_mov_b64 s[4:5], 0",
        "v_add_u32_e32 v1, 1, v1",                       # 0x1004: loop body
        "s_andn2_b64 exec, exec, s[4:5]",
        "s_cbranch_execnz 65533 <kernel+0x4>"]


def test_copy_after_divergent_loop_exit_is_found():
    text = _asm(LOOP + ["v_accvgpr_write_b32 a0, v1", "s_or_b64 exec, exec, s[4:5]",
                        "v_mov_b32_e32 v2, v1", "s_endpgm"])
    found = C.exec_zero_writes(text)
    assert [f[2] for f in found] == ["v_accvgpr_write_b32 a0, v1"]


def test_copy_after_exec_restore_is_fine():
    text = _asm(LOOP + ["s_or_b64 exec, exec, s[4:5]", "v_accvgpr_write_b32 a0, v1",
                        "v_writelane_b32 v3, s0, 1", "s_endpgm"])
    assert C.exec_zero_writes(text) == []


def test_lane_addressed_instructions_and_branch_targets_are_fine():
    # v_writelane ignores exec; a block that a branch or a far jump enters is
    # reached with lanes active
    text = _asm(LOOP + ["v_writelane_b32 v3, s0, 1", "s_or_b64 exec, exec, s[4:5]",
                        "s_branch 2 <kernel+0x2c>",
                        "s_cbranch_execnz 2 <kernel+0x2c>",
                        "v_cndmask_b32_e64 v2, 0, 1, s[4:5]",
                        "s_getpc_b64 s[98:99]", "s_add_u32 s98, s98, 0xffffffec",
                        "s_addc_u32 s99, s99, -1", "s_setpc_b64 s[98:99]", "s_endpgm"])
    # the v_cndmask at 0x1020 follows the second execnz; s_getpc at 0x1024
    # yields 0x1028, so an offset of -8 lands the far jump on the v_cndmask
    # (entered with lanes active) and -20 lands it on 0x1014
    text = text.replace("0xffffffec", "0xfffffff8")
    assert C.exec_zero_writes(text) == []
    assert [f[2] for f in C.exec_zero_writes(text.replace("0xfffffff8", "0xffffffec"))] == [
        "v_cndmask_b32_e64 v2, 0, 1, s[4:5]"]


def test_address_plus_register_is_not_followed():
    # s_getpc followed by a register offset (a table address, say) has no
    # known value: no jump target is taken from it, and reading it does not
    # fail
    text = _asm(LOOP + ["s_getpc_b64 s[12:13]", "s_add_u32 s12, s12, s14",
                        "s_addc_u32 s13, s13, 0", "s_setpc_b64 s[12:13]",
                        "v_mov_b32_e32 v2, v1", "s_endpgm"])
    assert C.exec_zero_writes(text) == []
    text = _asm(LOOP + ["s_getpc_b64 s[12:13]", "s_add_u32 s12, s12, s14",
                        "v_mov_b32_e32 v2, v1", "s_or_b64 exec, exec, s[4:5]", "s_endpgm"])
    assert [f[2] for f in C.exec_zero_writes(text)] == ["v_mov_b32_e32 v2, v1"]


@pytest.mark.skipif(not (C.LLVM_BIN / "llvm-objdump").exists(), reason="llvm-objdump absent")
def test_built_library_has_no_vector_writes_with_exec_zero():
    library = Path(__file__).resolve().parents[1] / "duck_gym_amd" / "libduck_hip.so"
    if not library.exists():
        pytest.skip("library not built")
    text = C.disassemble(library)
    assert "advanceKernel" in text
    assert C.exec_zero_writes(text) == []


def test_scalar_adds_to_non_sgpr_destinations_are_skipped():
    # s_add_u32 / s_addc_u32 on vcc_lo, ttmp or m0 are no half of a far jump:
    # the tracker skips them instead of misreading or failing on them
    lines = LOOP + ["s_add_u32 vcc_lo, vcc_lo, 4", "s_addc_u32 vcc_hi, vcc_hi, 0",
                    "s_add_u32 ttmp4, ttmp4, 8", "s_add_u32 m0, m0, 16",
                    "v_accvgpr_write_b32 a0, v1", "s_or_b64 exec, exec, s[4:5]", "s_endpgm"]
    assert [f[2] for f in C.exec_zero_writes(_asm(lines))] == ["v_accvgpr_write_b32 a0, v1"]
    # an m0 add after s_getpc of s[0:1] does not move the s0 pair's offset
    far = _asm(LOOP + ["v_cndmask_b32_e64 v2, 0, 1, s[4:5]",
                       "s_getpc_b64 s[0:1]", "s_add_u32 m0, m0, 0x100",
                       "s_add_u32 s0, s0, 0xfffffff8", "s_addc_u32 s1, s1, -1",
                       "s_setpc_b64 s[0:1]", "s_endpgm"])
    # s_getpc at 0x1014 yields 0x1018; -8 lands on the v_cndmask at 0x1010
    assert C.exec_zero_writes(far) == []


def test_scalar_cache_writes_are_found():
    text = _asm(["s_load_dwordx2 s[0:1], s[4:5], 0x0", "s_store_dword s2, s[0:1], 0x10",
                 "s_atomic_add s3, s[0:1], 0x0", "s_dcache_wb", "global_store_dword v0, v1, s[0:1]",
                 "s_endpgm"])
    assert C.scalar_writes(text) == ["s_store_dword", "s_atomic_add", "s_dcache_wb"]
    assert C.scalar_writes(_asm(LOOP + ["s_endpgm"])) == []
