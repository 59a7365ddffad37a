"""The q8 tier's int8 grouped GEMM (k_gemm_i8 / gemm_i8_body / launch_gemm_i8 in
eureka-engine_amd/csrc/moe_gemm.hip, driven by moe_q8_gemm in eureka-engine_amd/csrc/moe_q8.hip), its
index arithmetic restated on the host and run over every block, lane and 32-column block of real tile
lists: every q8_1 activation read stays inside its row and buffer, every {d, s} read inside the block
scales, every weight read inside its expert's row (byte ranges of the decoders from test_bounds) and the
expert stack, every LDS index inside the 64 x 32 {d, s} stage, every store inside the output, and every
(slot, output column) written exactly once. Shapes: config 1's 16- and 2048-token chunks, Zipf-skewed
64-token batches, config 5's 513-token batch with 512 experts, and the shared expert (no tile list).
A change to the kernel's addressing must be mirrored here.
"""
import numpy as np
import pytest

from test_bounds import BLK, i8_q6_reads, i8_reads

BM, QG_CH = 64, 32
FM_Q8_0, FM_Q4_K, FM_Q6_K, FM_Q5_K = 1, 3, 4, 9


def rbytes(fm, cols):
    b_, n = BLK[fm]
    return cols // n * b_


def launch_ok(fm, K, N, mode):
    """launch_gemm_i8's argument checks"""
    nf = 128 if mode == 0 else 256
    return K % 32 == 0 and N % nf == 0 and (fm == FM_Q8_0 or K % 256 == 0)


def weight_reads(fm, b, h):
    """byte ranges one lane reads of one weight row for 32-column block b"""
    if fm == FM_Q6_K:
        return [r for k in (0, 1) for r in i8_q6_reads(b, k, h)]
    return i8_reads(fm, b, h)


def check(fm, ne, T, nk, K, N, mode, tiles=True, seed=0, skew=None, fused=False):
    assert launch_ok(fm, K, N, mode)
    rng = np.random.default_rng(seed)
    n = T * nk
    nb = K // 32
    rb = rbytes(fm, K)
    if tiles:
        p = np.ones(ne) if skew is None else 1.0 / np.arange(1, ne + 1) ** skew
        p /= p.sum()
        ids = np.stack([rng.choice(ne, nk, replace=False, p=p) for _ in range(T)]).ravel()
        cnt = np.bincount(ids, minlength=ne)
        off = np.concatenate([[0], np.cumsum(cnt)])
        tl = [(e, k) for e in range(ne) for k in range((cnt[e] + BM - 1) // BM)]
        maxt = n // BM + ne + 1  # moe_q8_gemm's grid bound
        assert len(tl) <= maxt
        xmap = rng.integers(0, T, n) if mode == 0 else None  # gate / up reads token rows, down slot rows
        arows = T if mode == 0 else n
        slots = n
        nexp = ne
    else:
        maxt = (T + BM - 1) // BM
        tl, xmap = None, None
        arows = slots = T
        nexp = 1
    # the stack: ne experts of N rows (gate / up fused: 2 N rows, the up half after the gate half)
    es = (2 if fused else 1) * N * rb
    stack = nexp * es
    NT = N // (128 if mode == 0 else 256)
    ntl = len(tl) if tiles else maxt
    C = (ntl + 7) // 8
    nblk = 8 * NT * ((maxt + 7) // 8)
    tid = np.arange(256)
    w, l = tid >> 6, tid & 63
    h, lr = l >> 5, l & 31
    seen = np.zeros((ntl, NT), np.int32)
    written = np.zeros((slots, N), np.int32)
    lane_reads = {hh: [r for b in range(nb) for r in weight_reads(fm, b, hh)] for hh in (0, 1)}
    for hh in (0, 1):
        for s, e in lane_reads[hh]:
            assert 0 <= s < e <= rb, (fm, K, hh, s, e, rb)
    for blk in range(nblk):
        q = blk >> 3
        ntile = q % NT
        tile = (blk & 7) * C + q // NT
        if q // NT >= C or tile >= ntl:
            continue
        seen[tile, ntile] += 1
        if tiles:
            e, k = tl[tile]
            m0, base, M = k * BM, off[e], off[e + 1] - off[e]
        else:
            e, m0, base, M = 0, tile * BM, 0, T
        live = M - m0
        assert 0 < live and 0 <= e < nexp
        NL = 1 if live <= 32 else 2
        # activation rows: slot base + m0 + min(32 mf + lr, live - 1), 16 bytes at 16 h + 32 b (Q6_K: 8 at
        # 8 h + 32 b and 8 h + 32 b + 16)
        for mf in range(NL):
            slot = base + m0 + np.minimum(32 * mf + lr, live - 1)
            assert (slot >= base).all() and (slot < base + M).all() and (slot < slots).all()
            src = xmap[slot] if xmap is not None else slot
            assert (src < arows).all()
            if fm == FM_Q6_K:
                lo = np.minimum(8 * h, 8 * h + 16)
                hi = 8 * h + 32 * (nb - 1) + 16 + 8
            else:
                lo, hi = 16 * h, 16 * h + 32 * (nb - 1) + 16
            assert (lo >= 0).all() and (hi <= K).all() and ((src * K + hi) <= arows * K).all()
            assert ((16 * h) % 16 == 0).all() and K % 16 == 0  # i32x4 loads: 16-byte aligned rows
        # {d, s} staging: chunk c0, i < 64 cn, row min(i % 64, live - 1)
        for c0 in range(0, nb, QG_CH):
            cn = min(QG_CH, nb - c0)
            i = np.arange(64 * cn)
            r = np.minimum(i % 64, live - 1)
            slot = base + m0 + r
            src = xmap[slot] if xmap is not None else slot
            ad = src * nb + c0 + i // 64
            assert (ad < arows * nb).all() and (i < 64 * QG_CH).all()
            for bi in (0, cn - 1):
                for mf in range(NL):
                    for ii in range(16):
                        li = bi * 64 + 32 * mf + 8 * (ii >> 2) + 4 * h + (ii & 3)
                        assert (li < 64 * cn).all()
                        # the {d, s} of the row the MFMA puts in accumulator ii is that row's
                        row = 32 * mf + 8 * (ii >> 2) + 4 * h + (ii & 3)
                        assert (li % 64 == row).all()
        # weight rows of this lane
        if mode == 0:
            f = ntile * 128 + 32 * w + lr
            r0, r1 = f, f + (N if fused else 0)  # W1 = W0 + N rows when fused, else its own stack
            assert (f < N).all()
        else:
            r0 = ntile * 256 + 64 * w + lr
            r1 = r0 + 32
            assert (r1 < N).all()
        for rr in (r0, r1):
            start = e * es + rr * rb
            for s, end in lane_reads[0] + lane_reads[1]:
                assert ((start + end) <= stack).all() and ((start + s) >= e * es).all()
            assert ((rr + 1) * rb <= es).all()
        # epilogue
        for mf in range(NL):
            for ii in range(16):
                row = 32 * mf + 8 * (ii >> 2) + 4 * h + (ii & 3)
                ok = m0 + row < M
                s = base + m0 + row
                assert (s[ok] < slots).all()
                if mode == 0:
                    np.add.at(written, (s[ok], (ntile * 128 + 32 * w + lr)[ok]), 1)
                else:
                    for bb in range(2):
                        np.add.at(written, (s[ok], (ntile * 256 + 64 * w + 32 * bb + lr)[ok]), 1)
    assert (seen == 1).all()
    assert (written == 1).all(), (written.min(), written.max())


@pytest.mark.parametrize("args", [
    # config 1 (128 experts top 8, dm 2048, ef 768), Q8_0 and K-quants, 16 and 2048 tokens
    dict(fm=FM_Q8_0, ne=128, T=16, nk=8, K=2048, N=768, mode=0),
    dict(fm=FM_Q8_0, ne=128, T=16, nk=8, K=768, N=2048, mode=1),
    dict(fm=FM_Q8_0, ne=128, T=2048, nk=8, K=2048, N=768, mode=0, fused=True),
    dict(fm=FM_Q8_0, ne=128, T=2048, nk=8, K=768, N=2048, mode=1),
    dict(fm=FM_Q4_K, ne=128, T=64, nk=8, K=2048, N=768, mode=0, skew=1.1),
    dict(fm=FM_Q6_K, ne=128, T=64, nk=8, K=768, N=2048, mode=1, skew=1.1),
    dict(fm=FM_Q5_K, ne=128, T=40, nk=8, K=2048, N=768, mode=0),
    # config 5: 512 experts top 10, ef 512, 513 tokens
    dict(fm=FM_Q4_K, ne=512, T=513, nk=10, K=2048, N=512, mode=0, skew=1.1),
    dict(fm=FM_Q6_K, ne=512, T=513, nk=10, K=512, N=2048, mode=1, skew=1.1),
    # the shared expert: no tile list, M = T
    dict(fm=FM_Q8_0, ne=1, T=513, nk=1, K=2048, N=512, mode=0, tiles=False),
    dict(fm=FM_Q6_K, ne=1, T=161, nk=1, K=512, N=2048, mode=1, tiles=False),
])
def test_int8_gemm_indices_in_range(args):
    check(**args)


def test_launch_refuses_k_quant_rows_not_whole_super_blocks():
    """K-quant rows of K % 256 != 0 are refused by launch_gemm_i8; moe_q8_gemm must then not be chosen
    (q8_gemm_ok requires ef % 256 for K-quant down stacks), else the layer would end in an error"""
    assert not launch_ok(FM_Q4_K, 384, 2048, 1)
    assert launch_ok(FM_Q8_0, 384, 2048, 1)


def test_the_control_catches_a_stage_index_past_the_chunk():
    """the control: a {d, s} read with the chunk stride of 32 instead of 64 rows would name another
    slot's scales, and the row check above fails on it"""
    h = np.arange(64) >> 5
    li = 1 * 32 + 8 * 1 + 4 * h + 1
    assert not (li % 64 == 32 * 0 + 8 * 1 + 4 * h + 1).all()
