"""The device code carries no wide-store data hazard and no accumulator access
too close to an inline-asm MFMA (gonano_amd/isa_check).  Wide stores:
no store of more than 8 bytes is followed directly by a VALU write to its
data registers.  The scanner itself is checked on hand-written assembly:
the buffer-store case measured on MI355X, the global-store form, a write
to the address registers only (no hazard) and a 64-bit store (no hazard)."""
import pytest

from gonano_amd import isa_check


def _kernel(body: str) -> str:
    return "_ZN2gn1kEv:\n" + "\n".join("\t" + l for l in body.strip().split("\n")) + "\n.Lfunc_end0:\n"


def test_scanner_finds_the_measured_pattern():
    bad = _kernel("""
        buffer_store_dwordx4 v[18:21], v1, s[16:19], s5 offen
        v_or_b32_e32 v18, 0x6000, v4
    """)
    assert len(isa_check.scan(bad)) == 1
    bad_global = _kernel("""
        global_store_dwordx4 v[6:7], v[8:11], off
        v_mov_b32_e32 v10, 0
    """)
    assert len(isa_check.scan(bad_global)) == 1
    wide_dest = _kernel("""
        global_store_dwordx4 v[6:7], v[8:11], off
        v_mov_b64_e32 v[10:11], s[20:21]
    """)
    assert len(isa_check.scan(wide_dest)) == 1


def test_scanner_passes_safe_sequences():
    ok = _kernel("""
        global_store_dwordx4 v[6:7], v[8:11], off
        v_add_co_u32_e32 v6, vcc, 0x8000, v4
        buffer_store_dwordx4 v[18:21], v1, s[16:19], s5 offen
        s_nop 0
        v_or_b32_e32 v18, 0x6000, v4
        global_store_dwordx2 v[6:7], v[8:9], off
        v_mov_b32_e32 v8, 0
    """)
    assert isa_check.scan(ok) == []


def test_library_device_code_has_no_wide_store_hazard():
    try:
        isa_check.build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    assert isa_check.check() == []


def test_mfma_gap_scanner():
    """Accumulator reads after an inline-asm MFMA (which the compiler's
    hazard recognizer does not see): too close on a straight path and
    across a loop's back edge are found; 16 wait states pass; builtin MFMAs
    (the compiler's own business) are not checked."""
    asm_mfma = ";;#ASMSTART\nv_mfma_f32_16x16x4_f32 a[252:255], v1, v2, a[252:255]\n;;#ASMEND"
    straight = _kernel(asm_mfma + "\ns_add_i32 s1, s2, s3\nv_accvgpr_read_b32 v133, a255")
    assert len(isa_check.scan_mfma_gaps(straight)) == 1
    loop = _kernel(".LBB1_2:\ns_min_u32 s8, s30, s42\nv_accvgpr_read_b32 v133, a255\n" + asm_mfma +
                   "\ns_nop 3\ns_cbranch_scc0 .LBB1_2")
    assert len(isa_check.scan_mfma_gaps(loop)) == 1
    assert isa_check.scan_mfma_gaps(loop.replace("s_nop 3", "s_nop 7\n\ts_nop 7")) == []
    other_reg = _kernel(asm_mfma + "\nv_accvgpr_read_b32 v133, a3")
    assert isa_check.scan_mfma_gaps(other_reg) == []
    builtin = _kernel("v_mfma_f32_16x16x4_f32 a[252:255], v1, v2, a[252:255]\n"
                      "v_accvgpr_read_b32 v133, a255")
    assert isa_check.scan_mfma_gaps(builtin) == []
