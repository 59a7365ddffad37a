"""The one-token decode kernels (k_gu_dec, k_dn_dec, k_router in eureka-engine_amd/csrc/moe_decode.hip, launched
by decode_forward in eureka-engine_amd/csrc/llb_moe_hip.cpp), their address and LDS arithmetic restated on the
host and run over every block, wave and lane of real shapes: config 1, config 2, config 5 and the decode-test
shapes (every routed and shared format), separate and fused gate / up stacks, the first and the last expert.

Checked: every 16-byte PairChunks load lies inside its gate / up row and the stack; every byte the decoders
read from a staged row lies inside that row; the down launch's LDS-DMA window lies inside the expert's (or
the shared expert's) down rows and fits its staging area; the gate / up launch's down-row touch stays inside
the rows it is meant for (a control shows the earlier lower bound read before the stack); every LDS index
lies below the launch's LDS size, which is below the 160 KB a CU holds. A change to the kernels' addressing
must be mirrored here.
"""
import numpy as np
import pytest

import eureka_moe as em

FM_Q8_0, FM_Q4_K, FM_Q6_K, FM_Q5_K = 1, 3, 4, 9
BLK = {FM_Q8_0: (34, 32), FM_Q4_K: (144, 256), FM_Q5_K: (176, 256), FM_Q6_K: (210, 256)}
LDS_CU = 160 * 1024


def rbytes(fm, cols):
    b, n = BLK[fm]
    return cols // n * b


# ---- moe_decode.hip constants
DEC_DM, GU_WAVES, DN_RB = 2048, 16, 8
DEC_XS = (DEC_DM + DEC_DM // 16) * 4
DEC_TK = 64 * 4 + 64 * 8
DEC_GU = 32 * 2 * 4
DEC_LV = 2 * (DEC_DM // 4) * 4
TKB_LDS = 512 * 8 + 128 * 8 + 1024 + 64 * 4 + 64 * 8
DN_PART = DN_RB * 16 * 4


def xpad(c):
    return c + 4 * (c >> 6)


def gu_lds(rb):
    return DEC_XS + DEC_TK + DEC_GU + TKB_LDS + GU_WAVES * (2 * rb + DEC_LV)


def leaf_col(F, q, i):
    if F == FM_Q6_K:
        return 256 * (q >> 2) + 128 * ((q >> 1) & 1) + 32 * (q & 1) + (4 * i if i < 8 else 64 + 4 * (i - 8))
    return 64 * q + 4 * i


def leaves64_reads(F, q):
    """byte ranges (start, end) leaves64<F> reads of a row for 64-column group q"""
    if F == FM_Q4_K:
        B, g = 144 * (q >> 2), q & 3
        return [(B, B + 16), (B + 16 + 32 * g, B + 32 + 32 * g), (B + 32 + 32 * g, B + 48 + 32 * g)]
    if F == FM_Q5_K:
        B, g = 176 * (q >> 2), q & 3
        return [(B, B + 16), (B + 16, B + 32), (B + 32, B + 48), (B + 48 + 32 * g, B + 64 + 32 * g),
                (B + 64 + 32 * g, B + 80 + 32 * g)]
    if F == FM_Q6_K:
        B, n, a = 210 * (q >> 2), (q >> 1) & 1, q & 1
        o = B + 64 * n + 32 * a
        return [(o, o + 16), (o + 16, o + 32), (B + 128 + 32 * n, B + 144 + 32 * n),
                (B + 144 + 32 * n, B + 160 + 32 * n), (B + 192 + 8 * n + 2 * a, B + 194 + 8 * n + 2 * a),
                (B + 196 + 8 * n + 2 * a, B + 198 + 8 * n + 2 * a), (B + 208, B + 210)]
    B = 68 * q  # Q8_0: blocks 2 q, 2 q + 1
    r = []
    for b in range(2):
        K = B + 34 * b
        r += [(K, K + 2), (K + 2, K + 18), (K + 18, K + 34)]
    return r


def q8_block_reads(F, b):
    """bytes blk_q8<F> reads of a row for 32-column block b (moe_q8dot.h): the block's own bytes"""
    if F == FM_Q8_0:
        return [(34 * b, 34 * b + 34)]
    bb, n = BLK[F]
    s = 32 * b // n
    return [(bb * s, bb * s + bb)]


def test_decoders_read_inside_the_row():
    """for cols 256 .. 4096 every group / block a lane decodes lies inside the row"""
    for F in BLK:
        for cols in (256, 512, 768, 2048, 4096):
            rb = rbytes(F, cols)
            for q in range(cols // 64):
                for s, e in leaves64_reads(F, q):
                    assert 0 <= s < e <= rb, (F, cols, q, s, e)
                for bq in (2 * q, 2 * q + 1):
                    for s, e in q8_block_reads(F, bq):
                        assert 0 <= s < e <= rb
                for i in range(16):
                    c = leaf_col(F, q, i)
                    assert 0 <= c and c + 4 <= cols  # the leaf's activations
    # the routed leaves of one 2048-column row in moe_dot's place: leaf index leaf_col / 4 covers
    # 0 .. 511 once (put_leaves writes each float4 once)
    for F in BLK:
        seen = np.zeros(512, np.int32)
        for q in range(32):
            for i in range(16):
                seen[leaf_col(F, q, i) // 4] += 1
        assert (seen == 1).all(), F


# ---- shapes

def dec_ok(s, base_g=0x10000, base_d=0x900010):
    """decode_forward's admission (dec_ok), from the shape alone (bases 16-aligned)"""
    if s.dm != 2048 or s.fg != s.fu or s.nk + (1 if s.sf else 0) > 16 or s.ef % 128 or s.ef > 4096:
        return False
    if s.sf > 15 * (s.nk * s.ef // 16):
        return False
    if s.sf and (s.sf % 128 or s.sf > 4096):
        return False
    return True


SHAPES = [em.SHAPES[n] for n in ("c1", "c2", "c1k", "c5")] + [
    em.Shape(2048, 32, 4, 256, 256, em.Q4_K, em.Q4_K, em.Q6_K),
    em.Shape(2048, 16, 2, 512, 0, em.Q8_0, em.Q8_0, em.Q8_0),
    em.Shape(2048, 64, 6, 256, 512, em.Q5_K, em.Q5_K, em.Q5_K, fsg=em.Q5_K, fsu=em.Q5_K, fsd=em.Q4_K),
    em.Shape(2048, 24, 3, 256, 256, em.Q6_K, em.Q6_K, em.Q5_K, fsg=em.Q6_K, fsu=em.Q6_K, fsd=em.Q6_K),
    em.Shape(2048, 16, 4, 512, 256, em.Q8_0, em.Q8_0, em.Q4_K, fsg=em.Q4_K, fsu=em.Q4_K, fsd=em.Q5_K),
    em.Shape(2048, 20, 15, 768, 0, em.Q4_K, em.Q4_K, em.Q6_K),
]
IDS = lambda s: sorted({0, s.ne - 1, s.ne // 2})  # noqa: E731  (experts a slot may hold)


def pair_chunk_ranges(RB, row_g, row_u, L):
    """PairChunks<RB>::load: 16-byte loads of lane L (all k)"""
    CP = 2 * (RB // 16)
    NR = (CP + 63) // 64
    out = []
    for k in range(NR):
        c = min(L + 64 * k, CP - 1)
        a = row_g + 16 * c if c < RB // 16 else row_u + 16 * (c - RB // 16)
        out.append((a, a + 16, c))
    return out


@pytest.mark.parametrize("si", range(len(SHAPES)))
@pytest.mark.parametrize("fused", [False, True])
def test_gu_dec_loads_inside_rows_and_stacks(si, fused):
    s = SHAPES[si]
    assert dec_ok(s)
    RB, RBS = rbytes(s.fg, 2048), rbytes(s.fsg, 2048) if s.sf else 0
    assert RB % 16 == 0 and RBS % 16 == 0  # the chunking needs it
    G = 0x10000
    es = (2 if fused else 1) * s.ef * RB
    U = G + s.ef * RB if fused else 0x40000000
    gbytes = s.ne * es
    nrb = s.nk * s.ef // GU_WAVES
    bps = s.ef // GU_WAVES
    assert not (s.sf and s.sf > 15 * nrb)
    for blk in range(nrb):
        slot, f0 = blk // bps, (blk % bps) * GU_WAVES
        assert slot < s.nk
        for w in range(GU_WAVES):
            f = f0 + w
            assert f < s.ef
            for e in IDS(s):
                rg, ru = G + e * es + f * RB, U + e * es + f * RB
                for L in range(64):
                    for a, b, c in pair_chunk_ranges(RB, rg, ru, L):
                        row = rg if c < RB // 16 else ru
                        assert row <= a and b <= row + RB
                        base = G if (fused or c < RB // 16) else U
                        assert base <= a and b <= base + gbytes
                        if fused:
                            assert G <= a and b <= G + gbytes
            # the shared expert's rows (waves 1 ..)
            sfeat = blk + nrb * (w - 1)
            if s.sf and w >= 1 and sfeat < s.sf:
                SG, SU = 0x70000000, 0x78000000
                for L in range(64):
                    for a, b, c in pair_chunk_ranges(RBS, SG + sfeat * RBS, SU + sfeat * RBS, L):
                        bs = SG if c < RBS // 16 else SU
                        assert bs <= a and b <= bs + s.sf * RBS
    # every shared feature is taken by exactly one (block, wave)
    if s.sf:
        got = sorted(blk + nrb * (w - 1) for blk in range(nrb) for w in range(1, GU_WAVES) if blk + nrb * (w - 1) < s.sf)
        assert got == list(range(s.sf))
        # the SwiGLU epilogue's lanes 16 + k match the waves that computed them: ns per block
        for blk in range(nrb):
            ns = min(15, (s.sf - blk + nrb - 1) // nrb if s.sf > blk else 0)
            waves = [w for w in range(1, GU_WAVES) if blk + nrb * (w - 1) < s.sf]
            assert ns == len(waves) and waves == list(range(1, ns + 1))
    # every (slot, feature) of act is written once
    seen = np.zeros((s.nk, s.ef), np.int32)
    for blk in range(nrb):
        for L in range(16):
            seen[blk // bps, (blk % bps) * GU_WAVES + L] += 1
    assert (seen == 1).all()


def touch_addr(base, L, old=False):
    lo = base - (base & 127)
    return lo + 128 * L if (old or L != 0) else base


@pytest.mark.parametrize("si", range(len(SHAPES)))
def test_gu_dec_down_touch_stays_in_the_rows(si):
    """the touch of block b3's down rows: lines of [base, base + DN_RB rb) only; waves without a task, and
    blocks past the down grid, touch the first dword of the stack. D 16-aligned (dec_ok), not 128-aligned"""
    s = SHAPES[si]
    rbd = rbytes(s.fd, s.ef)
    rbs = rbytes(s.fsd, s.sf) if s.sf else 0
    D, SD = 0x900010, 0x7F000010
    dbytes = s.ne * s.dm * rbd
    ndb = (s.dm + 7) // 8
    nrb = s.nk * s.ef // GU_WAVES
    for blk in range(nrb):
        b3 = blk if blk < ndb else 0
        for w in range(GU_WAVES):
            sh = bool(s.sf) and w == s.nk
            rb = rbs if sh else rbd
            for e in IDS(s):
                base = SD + DN_RB * b3 * rb if sh else D + (e * s.dm + DN_RB * b3) * rb
                end = base + DN_RB * rb
                live_w = w < s.nk + (1 if s.sf else 0)
                for L in range(64):
                    p = touch_addr(base, L)
                    live = live_w and p + 4 <= end
                    a = p if live else D
                    if live:
                        assert base <= a and a + 4 <= end
                    lo_buf, hi_buf = (SD, SD + s.dm * rbs) if (sh and live) else (D, D + dbytes)
                    assert lo_buf <= a and a + 4 <= hi_buf, (blk, w, e, L)
    # control: the earlier lower bound (line 0 at base rounded down to 128) read before the stack
    base = D + (0 * s.dm + 0) * rbd
    assert touch_addr(base, 0, old=True) < D


def dn_dec_lds(nk, ef, sf, rbd, rbs, dm, shared, q8):
    nt = nk + (1 if shared else 0)
    cm = 256 if q8 else 128
    if nt > 16 or ef % cm or ef > 4096 or (shared and (sf % cm or sf > 4096)) or dm % DN_RB:
        return None
    rbmax = max(rbd, rbs)
    sb = (DN_RB * rbmax + 32 + 15) & ~15
    cmax = max(ef, sf)
    xb = (cmax + cmax // 32 * 8 + 15) & ~15 if q8 else (cmax + cmax // 16) * 4
    lds = DN_PART + nt * (sb + xb + 4096)
    if lds > LDS_CU - 256:
        return None
    return lds, sb, xb


@pytest.mark.parametrize("si", range(len(SHAPES)))
@pytest.mark.parametrize("q8", [False, True])
def test_dn_dec_window_and_lds(si, q8):
    s = SHAPES[si]
    rbd = rbytes(s.fd, s.ef)
    rbs = rbytes(s.fsd, s.sf) if s.sf else 0
    r = dn_dec_lds(s.nk, s.ef, s.sf, rbd, rbs, s.dm, bool(s.sf), q8)
    if r is None:
        assert not q8, "the q8 decode needs the down launch (dec_q8_ok)"
        return  # the exact tier falls back to the general down kernel
    lds, sb, xb = r
    assert lds + 64 <= LDS_CU  # and 64 bytes of static LDS (wsh)
    D, SD = 0x900010, 0x7F000010
    assert (s.dm * rbd) % 16 == 0 and (s.dm * rbs) % 16 == 0  # stacks a multiple of 16 bytes
    nt = s.nk + (1 if s.sf else 0)
    for blk in range((s.dm + DN_RB - 1) // DN_RB):
        r0 = blk * DN_RB
        nrow = min(DN_RB, s.dm - r0)
        for w in range(nt):
            shared = bool(s.sf) and w == s.nk
            cols, rb = (s.sf, rbs) if shared else (s.ef, rbd)
            for e in IDS(s):
                base = SD + r0 * rb if shared else D + (e * s.dm + r0) * rb
                lo_buf, hi_buf = (SD, SD + s.dm * rbs) if shared else (D + e * s.dm * rbd, D + (e + 1) * s.dm * rbd)
                a16 = base & ~15
                b16 = (base + nrow * rb + 15) & ~15
                nch = (b16 - a16) // 16
                # the window: inside this expert's down rows (16-aligned stacks of whole 16-byte units)
                assert lo_buf <= a16 and b16 <= hi_buf, (blk, w, e)
                # the DMA writes stage + 16 c, c < nch; it fits the staging area
                assert nch * 16 <= sb
                # rows read from stage + (base - a16) + rr rb + (offset inside the row)
                assert (base - a16) + nrow * rb <= nch * 16
            # activations: padded floats or q8_1 codes + {d, s}
            if q8:
                assert cols % 256 == 0 and cols + cols // 32 * 8 <= xb
            else:
                assert (xpad(cols - 4) + 4) * 4 <= xb
            lpr, rpp = cols // 64, 64 // (cols // 64)
            assert lpr >= 1 and rpp >= 1
            if not q8:
                assert rpp * (cols // 4) * 4 <= 4096  # leaves of one pass
                assert all(32 * m + v < cols // 4 for m in [cols // 128 - 1] for v in [31])
            # part[(p0 + rl) * 16 + w]
            assert (nrow - 1) * 16 + w < DN_PART // 4
    assert s.nk <= 16  # wsh[16]


@pytest.mark.parametrize("si", range(len(SHAPES)))
def test_gu_dec_lds(si):
    """k_gu_dec's LDS: x (padded) | ids + candidates | gate / up dots | topk_block | 16 waves x (staged pair +
    leaves); every index inside its region, the total below the CU's 160 KB"""
    s = SHAPES[si]
    RB = rbytes(s.fg, 2048)
    RBX = max(RB, rbytes(s.fsg, 2048) if s.sf else 0)
    assert gu_lds(RBX) <= LDS_CU
    # x: xpad(4 t) + 4 floats, t < 512
    assert (xpad(4 * 511) + 4) * 4 <= DEC_XS
    # q8: codes [2048] bytes then {d, s} [64] at byte 2048
    assert 2048 + 64 * 8 <= DEC_XS
    # gus: index 2 (16 + w - 1) + 1 for w <= 15, and the epilogue's 2 L + 1 for L < 16 + 15
    assert (2 * (16 + 15 - 1) + 1 + 1) * 4 <= DEC_GU and (2 * 30 + 1 + 1) * 4 <= DEC_GU
    # topk_block: key [512] u64 | cand [8][16] u64 | cnt [1024] u8 | red [64] f32 | sid [64] | sp [64]
    for NP in (256, 512):
        NW, PK = NP // 64, 1024 // NP
        assert max(sg * NP + j for sg in range(PK) for j in range(NP)) < 1024
        assert 16 * NW * NW <= 1024 and (NW - 1) * 16 + 15 < 128
        assert 16 + (NP - 1) // 32 < 64
    assert 512 * 8 + 128 * 8 + 1024 + 64 * 4 + 64 * 4 + 64 * 4 == TKB_LDS
    # the wave's stage: 2 rows of up to RBX bytes; the leaves: 2 x 512 floats
    assert 2 * (2048 // 4) * 4 == DEC_LV
    for F in {s.fg, s.fsg if s.sf else s.fg}:
        rb = rbytes(F, 2048)
        for L in range(64):
            h, q = L >> 5, L & 31
            for a, b in leaves64_reads(F, q):
                assert h * rb + b <= 2 * RBX
            for i in (0, 4, 8, 12):
                assert h * 512 + leaf_col(F, q, i) // 4 + 4 <= 1024


def test_router_reads_inside_rows():
    """k_router<NQ>: lane L of wave w loads float4 64 q + L, q in [QW w, QW w + QW), only below cols / 4"""
    for cols, nq in ((2048, 8), (4096, 16), (8192, 32), (1536, 8)):
        nl4, qw = cols // 4, nq // 4
        seen = np.zeros(nl4, np.int32)
        for w in range(4):
            for k in range(qw):
                q = qw * w + k
                for L in range(64):
                    if 64 * q + L < nl4:
                        seen[64 * q + L] += 1
        assert (seen == 1).all(), cols
