"""Build check: no MFMA of the library sits in an EXEC-masked block that the
GPU would run with EXEC = 0 (MFMAs ignore EXEC, so such a block overwrites
its accumulator), and no kernel spills to scratch beyond the listed spills.
The scanners are pinned on hand-written assembly first."""

import shutil

import pytest

from cxldsagr_amd.csrc import isa_check

GUARDED = """
_Zkernel:
    v_cmp_ne_u32_e32 vcc, 0, v0
    s_and_saveexec_b64 s[0:1], vcc
    s_xor_b64 s[2:3], exec, s[0:1]
    s_cbranch_execz .LBB0_2
    v_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], v[0:3]
.LBB0_2:
    s_or_b64 exec, exec, s[0:1]
    v_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], v[0:3]
"""

# The form that gave wrong results: an if / else on a lane-derived value, each
# side one MFMA into the same accumulator, no skip on either side.
IF_ELSE_UNGUARDED = """
_Zkernel:
    v_cmp_ne_u32_e64 s[2:3], 0, v9
    s_and_saveexec_b64 s[4:5], s[2:3]
    s_xor_b64 s[4:5], exec, s[4:5]
    v_mov_b32_e32 v10, 0x3f803f80
    v_mfma_f32_16x16x32_bf16 v[42:45], v[10:13], v[194:197], v[2:5]
    s_andn2_saveexec_b64 s[4:5], s[4:5]
    v_mov_b32_e32 v10, 0x3f803f80
    v_mfma_f32_16x16x32_bf16 v[42:45], v[10:13], a[0:3], v[2:5]
    s_or_b64 exec, exec, s[4:5]
"""

# A skip that comes after the side's first vector instruction does not count,
# and the else side of a compiled if / else (s_or_saveexec + s_xor exec) needs
# its own skip.
LATE_SKIP_AND_ELSE = """
_Zkernel:
    s_and_saveexec_b64 s[4:5], vcc
    v_mov_b32_e32 v1, 0
    s_cbranch_execz .LBB0_1
    v_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]
.LBB0_1:
    s_or_saveexec_b64 s[4:5], s[4:5]
    s_xor_b64 exec, exec, s[4:5]
    s_cbranch_execz .LBB0_2
    v_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]
.LBB0_2:
    s_or_b64 exec, exec, s[4:5]
"""

SCALAR_BRANCH = """
_Zkernel:
    v_readfirstlane_b32 s2, v214
    s_bitcmp0_b32 s2, 0
    s_cbranch_scc1 .LBB0_64
    v_mfma_f32_16x16x32_bf16 v[42:45], v[10:13], v[198:201], v[2:5]
.LBB0_64:
    v_mfma_f32_16x16x32_bf16 v[42:45], v[10:13], v[194:197], v[2:5]
"""


def test_scanner_accepts_skipped_sides_and_scalar_branches():
    assert isa_check.unguarded_mfma(GUARDED) == []
    assert isa_check.unguarded_mfma(SCALAR_BRANCH) == []


def test_scanner_flags_unskipped_sides():
    found = isa_check.unguarded_mfma(IF_ELSE_UNGUARDED)
    # Line numbers count the snippet's leading empty line.
    assert [(f, line) for f, line, _ in found] == [("_Zkernel", 7), ("_Zkernel", 10)]
    found = isa_check.unguarded_mfma(LATE_SKIP_AND_ELSE)
    assert [line for _, line, _ in found] == [6]


KERNEL_DESCRIPTORS = """
.amdhsa_kernel _ZN3dsa12_GLOBAL__N_1fastE
    .amdhsa_private_segment_fixed_size 0
.end_amdhsa_kernel
.amdhsa_kernel _ZN3dsa12_GLOBAL__N_19topk_rowsILi17EEEvPKf
    .amdhsa_private_segment_fixed_size 28
.end_amdhsa_kernel
.amdhsa_kernel _ZN3dsa12_GLOBAL__N_114layer_prologueE
    .amdhsa_private_segment_fixed_size 212
.end_amdhsa_kernel
"""


def test_scratch_report_names_each_spilling_kernel():
    found = isa_check.scratch_bytes(KERNEL_DESCRIPTORS)
    assert found == {"_ZN3dsa12_GLOBAL__N_19topk_rowsILi17EEEvPKf": 28,
                     "_ZN3dsa12_GLOBAL__N_114layer_prologueE": 212}
    # The listed spill passes only at its listed size.
    assert isa_check.unknown_spills(found) == {"_ZN3dsa12_GLOBAL__N_114layer_prologueE": 212}
    assert isa_check.unknown_spills({"_ZN3dsa12_GLOBAL__N_19topk_rowsILi17EEEvPKf": 40}) != {}


@pytest.mark.skipif(shutil.which("hipcc") is None and not isa_check.build.Path("/opt/rocm/bin/hipcc").exists(),
                    reason="needs hipcc")
def test_library_has_no_mfma_in_unskipped_masked_blocks_and_no_new_spills():
    mfma, spills = isa_check.analyse()
    assert mfma == {}
    assert spills == {}
