"""The table row decode and pass_mail's admission check (host code of the C ABI, no GPU)."""
import ctypes as C

import numpy as np
import pytest

import eureka_moe as em

lib = em.load()


def c2_words(base_len=1 << 24):
    """a config-2 layer's 32 table words as tools/gguf2pack.c moe_sidecar_cuda writes them"""
    w = np.zeros(32, np.uint32)
    w[3] = 0x100000 | em.Q4_K << 28    # shared gate (Offs word 2)
    w[4] = 0x200000 | em.Q4_K << 28    # shared up
    w[5] = 0x300000 | em.Q6_K << 28    # shared down
    w[21] = 0x000400 | em.F32 << 28    # router
    w[22] = 0x200400 | em.F32 << 28    # shared gate row: right after the router's 256 x 2048 x 4 B
    w[26] = em.Q4_K | em.Q4_K << 4 | em.Q6_K << 8 | 1 << 13
    w[27], w[28], w[29], w[30] = 256, 512, 512, 8
    return w


def check(w, dm=2048, df=6144, ln=1 << 24):
    return lib.llb_moe_table_check(w.ctypes.data_as(C.POINTER(C.c_uint32)), dm, df, ln)


def test_decode_follows_llb_moe_run():
    w = c2_words()
    L = em.MoeLayer()
    assert lib.llb_moe_layer_from_table(w.ctypes.data_as(C.POINTER(C.c_uint32)), 2048, 0x10000000, 0xA000, 0xB000,
                                        0xC000, C.byref(L)) == 0
    assert (L.dm, L.ne, L.nk, L.ef, L.sf) == (2048, 256, 8, 512, 512)
    assert (L.fx & 15, L.fx >> 4 & 15, L.fx >> 8 & 15) == (em.Q4_K, em.Q4_K, em.Q6_K)
    assert (L.fsg, L.fsu, L.fsd) == (em.Q4_K, em.Q4_K, em.Q6_K)
    assert L.router == 0x10000400 and L.shgate == 0x10200400
    assert (L.SG, L.SU, L.SD) == (0x10100000, 0x10200000, 0x10300000)
    assert (L.G, L.U, L.D) == (0xA000, 0xB000, 0xC000)
    w[26] |= 1 << 12  # fused gate+up: U is G's second half, not a stack of its own
    assert lib.llb_moe_layer_from_table(w.ctypes.data_as(C.POINTER(C.c_uint32)), 2048, 0, 1, 2, 3, C.byref(L)) == 0
    assert L.U == 0


def test_admission_accepts_config_2():
    assert check(c2_words()) == 0
    w = c2_words()
    w[27] = 0
    assert check(w) == 0  # a dense layer: nothing to admit


@pytest.mark.parametrize("mut", ["nk>ne", "ef%256", "sf<256", "ef>df", "bit13", "fmt", "fused", "router fm",
                                 "ro%4", "router past len", "shgate past len", "nk=0"])
def test_admission_rejects_each_rule(mut):
    w = c2_words()
    if mut == "nk>ne": w[30] = 300
    if mut == "ef%256": w[28] = 640
    if mut == "sf<256": w[29] = 128
    if mut == "ef>df": w[28] = 8192
    if mut == "bit13": w[26] &= ~np.uint32(1 << 13)
    if mut == "fmt": w[26] = (w[26] & ~np.uint32(15)) | 5  # Q3_K is not an expert format here
    if mut == "fused": w[26] |= 1 << 12 | em.Q6_K << 4
    if mut == "router fm": w[21] = (w[21] & 0x0fffffff) | em.Q8_0 << 28
    if mut == "ro%4": w[21] += 2
    if mut == "router past len": w[21] = 0x0f000000 | em.F32 << 28
    if mut == "shgate past len": w[22] = 0x0ffffffc | em.F32 << 28
    if mut == "nk=0": w[30] = 0
    assert check(w) == 8
