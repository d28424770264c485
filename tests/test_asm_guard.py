"""The build-time guard of the large-shape GEMM's inline-assembly weight loads (minimax-h3-turbo_amd/asm_guard.py):
it passes the built code object, and it catches a planted copy, spill or reuse of an in-flight weight register in a
synthetic disassembly."""
import os

import pytest

import asm_guard

OBJ = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "minimax-h3-turbo_amd", "_build",
                   "h3k_gemm_w8p.o")
HEAD = "0000000000005500 <_ZN3h3k3w8p15gemm_w8p_kernelILi4ELi0ELb0EEEvPKal>:\n"


def dis(*body):
    return HEAD + "".join(f"\t{b}   // 0000: 00\n" for b in body)


LOAD = "buffer_load_dwordx4 v[8:11], v163, s[36:39], s55 offen offset:1024"


def test_clean_sequences_pass():
    ok = [dis(LOAD, "v_add_u32_e32 v1, v2, v3", "v_mfma_i32_32x32x32_i8 a[0:15], v[8:11], v[20:23], a[0:15]"),
          dis(LOAD, LOAD.replace("offset:1024", "offset:0")),
          dis(LOAD, "s_waitcnt vmcnt(0)", "scratch_store_dwordx4 off, v[8:11], off"),
          dis(LOAD, "buffer_load_dwordx4 v12, s[28:31], 0 offen lds", "v_mov_b32_e32 v12, 0")]
    for text in ok:
        assert asm_guard.violations(asm_guard.kernels_of_disassembly(text)) == []


@pytest.mark.parametrize("planted", ["scratch_store_dwordx4 off, v[8:11], off offset:16", "v_mov_b32_e32 v20, v9",
                                     "v_mov_b32_e32 v10, 0", "ds_read_b128 v[8:11], v141 offset:2048",
                                     "s_waitcnt vmcnt(4)"])
def test_a_touch_before_the_data_lands_fails(planted):
    text = dis(LOAD, planted, "v_mfma_i32_32x32x32_i8 a[0:15], v[8:11], v[20:23], a[0:15]")
    bad = asm_guard.violations(asm_guard.kernels_of_disassembly(text))
    if planted.startswith("s_waitcnt"):
        assert bad == []  # a partial wait is not a touch; the MFMA then reads the registers
    else:
        assert len(bad) == 1 and planted.split()[0] in bad[0]


def test_a_kernel_without_weight_loads_is_reported():
    assert asm_guard.violations(asm_guard.kernels_of_disassembly(dis("v_add_u32_e32 v1, v2, v3")))


@pytest.mark.skipif(not (os.path.exists(OBJ) and asm_guard.available()), reason="library not built here")
def test_the_built_object_passes():
    assert asm_guard.check_object(OBJ) == []
