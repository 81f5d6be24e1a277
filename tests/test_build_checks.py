"""The build's check of the global_load_lds hazard pad (oxmera_amd/build.py
check_dma_hazards): a VMEM read of an SGPR that a VALU instruction wrote
needs 5 wait states, so a DMA whose asm block carries the short pad
(s_nop 0) must not follow a VALU write of its base SGPRs that closely."""
from oxmera_amd.build import check_dma_hazards

DMA0 = "\ts_mov_b32 m0, s7\n\ts_nop 0\n\tglobal_load_lds_dwordx4 v1, s[2:3]\n"
DMA4 = "\ts_mov_b32 m0, s7\n\ts_nop 4\n\tglobal_load_lds_dwordx4 v1, s[2:3]\n"


def test_full_pad_after_readfirstlane_is_accepted():
    assert check_dma_hazards("\tv_readfirstlane_b32 s3, v3\n\tv_readfirstlane_b32 s2, v2\n" + DMA4) == []


def test_short_pad_after_a_full_pad_dma_is_accepted():
    asm = "\tv_readfirstlane_b32 s2, v2\n" + DMA4 + "\ts_add_i32 s7, s6, 0x1000\n" + DMA0
    assert check_dma_hazards(asm) == []


def test_short_pad_right_after_readfirstlane_is_refused():
    probs = check_dma_hazards("\tv_readfirstlane_b32 s3, v3\n" + DMA0)
    assert len(probs) == 1 and "VALU write" in probs[0]


def test_vop3_carry_out_into_the_base_is_refused():
    probs = check_dma_hazards("\tv_add_co_u32 v4, s[2:3], v1, v2\n\tv_mfma_f32_16x16x32_bf16 a[0:3], v[8:11], v[12:15], a[0:3]\n" + DMA0)
    assert len(probs) == 1


def test_write_of_other_sgprs_is_accepted_and_distance_counts_nops():
    assert check_dma_hazards("\tv_readfirstlane_b32 s9, v3\n" + DMA0) == []
    assert check_dma_hazards("\tv_readfirstlane_b32 s2, v3\n\ts_nop 4\n" + DMA0) == []
    assert check_dma_hazards("\tv_readfirstlane_b32 s2, v3\n\ts_nop 1\n" + DMA0) != []


def test_block_boundary_before_a_short_pad_is_refused():
    probs = check_dma_hazards(".LBB0_3:\n" + DMA0)
    assert len(probs) == 1 and "block boundary" in probs[0]


def test_unexpected_sequence_is_refused():
    assert check_dma_hazards("\ts_nop 0\n\tglobal_load_lds_dwordx4 v1, s[2:3]\n") != []
