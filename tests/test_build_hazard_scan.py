"""The build's scan for LDS-DMA copies that read an SGPR (or M0) a VALU instruction wrote fewer
than five wait states before (reels_amd/build.py lds_dma_hazards): the compiler inserts those wait
states for its own instructions but not around inline asm. Hand-written assembly snippets, the
copy in the form the kernels' inline asm takes (s_nop, then buffer_load_dwordx4 ... lds)."""
from reels_amd.build import lds_dma_hazards

HEAD = "_ZN5reels6kernelEv:\n"


def _asm(*lines):
    return HEAD + "\n".join("\t" + l for l in lines) + "\n"


def test_readlane_of_a_descriptor_word_one_wait_state_before_is_flagged():
    text = _asm("v_readlane_b32 s11, v252, 45",
                "s_mov_b32 m0, s3",
                ";;#ASMSTART",
                "s_nop 0",
                "buffer_load_dwordx4 v5, s[8:11], s14 offen lds",
                ";;#ASMEND")
    hits = lds_dma_hazards(text)
    assert len(hits) == 1 and hits[0][0] == "_ZN5reels6kernelEv" and "s11" in hits[0][2]


def test_readlane_of_the_offset_register_is_flagged():
    text = _asm("v_readfirstlane_b32 s14, v3", "s_nop 0",
                "buffer_load_dwordx4 v5, s[8:11], s14 offen lds")
    assert len(lds_dma_hazards(text)) == 1


def test_five_wait_states_clear_it():
    # s_nop 4 is five wait states
    text = _asm("v_readlane_b32 s11, v252, 45", "s_nop 4",
                "buffer_load_dwordx4 v5, s[8:11], s14 offen lds")
    assert lds_dma_hazards(text) == []
    # four instructions and one s_nop 0 between: five wait states too
    text = _asm("v_readlane_b32 s11, v252, 45", "v_add_u32_e32 v1, v2, v3",
                "v_add_u32_e32 v1, v2, v3", "s_mov_b32 s1, 0", "v_mov_b32_e32 v9, 0",
                "s_nop 0", "buffer_load_dwordx4 v5, s[8:11], s14 offen lds")
    assert lds_dma_hazards(text) == []


def test_salu_writes_and_unrelated_sgprs_are_not_flagged():
    text = _asm("s_mov_b32 s11, 0x20000", "v_readlane_b32 s20, v252, 3", "s_nop 0",
                "buffer_load_dwordx4 v5, s[8:11], s14 offen lds")
    assert lds_dma_hazards(text) == []


def test_valu_write_of_m0_is_flagged_and_loads_without_lds_are_ignored():
    text = _asm("v_readfirstlane_b32 m0, v7", "s_nop 0",
                "buffer_load_dwordx4 v5, s[8:11], s14 offen lds")
    assert len(lds_dma_hazards(text)) == 1
    text = _asm("v_readlane_b32 s11, v252, 45", "buffer_load_dwordx4 v[4:7], v5, s[8:11], 0 offen")
    assert lds_dma_hazards(text) == []
