"""The grouped GEMM's index arithmetic (k_moe_gemm3 and launch_moe_gemm in
eureka-engine_amd/csrc/moe_gemm.hip), restated on the host and run over every block, thread and k-tile
of real tile lists (read off the slot offsets by a wave scan, restated below): every global read stays inside its buffer (activation rows past a tile's slots
carry an offset past A's buffer bound, which the buffer load answers with zeros and no access), every
weight read inside its expert's rows and columns, every LDS access inside its stage, every store inside
the output, and every (slot, output column) written exactly once. Shapes: the 2048-token prefill,
Zipf-skewed 64-token batches, config 5's 513-token mixed batch, and the shared expert.
A change to the kernel's addressing must be mirrored here.
"""
import numpy as np
import pytest

MF, BK, LD = 2, 64, 72
BM = 32 * MF
STAGE = BM * LD  # halves


def check(ne, T, nk, K, N, mode, tiles=True, seed=0, skew=None):
    rng = np.random.default_rng(seed)
    n = T * nk
    if tiles:
        p = np.ones(ne) if skew is None else (1.0 / np.arange(1, ne + 1) ** skew)
        p /= p.sum()
        ids = np.stack([rng.choice(ne, nk, replace=False, p=p) for _ in range(T)]).ravel()
        cnt = np.bincount(ids, minlength=ne)
        off = np.concatenate([[0], np.cumsum(cnt)])
        tl = [(e, k) for e in range(ne) for k in range((cnt[e] + BM - 1) // BM)]
        maxt = n // BM + ne + 1  # the host's bound on the tile count (scratch and grid)
        assert len(tl) <= maxt, (len(tl), maxt)
        xmap = rng.integers(0, T, n)  # slot -> token (any map into [0, T))
        arows = T if mode == 0 else n
        slots = n
    else:
        maxt = (T + BM - 1) // BM
        tl = None
        arows = slots = T
    NF = 128 if mode == 0 else 256
    assert N % NF == 0 and K % BK == 0 and arows * K * 2 < 2**31
    NT = N // NF
    nblk = 8 * NT * ((maxt + 7) // 8)
    nkt = K // BK
    written = np.zeros((slots, N), np.int32)
    tid = np.arange(256)
    w, l = tid >> 6, tid & 63
    h, lr = l >> 5, l & 31
    bound = arows * K * 2
    ntl = len(tl) if tiles else (T + BM - 1) // BM
    C = (ntl + 7) // 8
    seen = np.zeros((ntl, NT), np.int32)
    for b in range(nblk):
        q, ntile = b >> 3, (b >> 3) % NT
        tile = (b & 7) * C + q // NT
        if q // NT >= C or tile >= ntl:
            continue
        seen[tile, ntile] += 1
        if tiles:
            e, k = tl[tile]
            m0, base, M = k * BM, off[e], off[e + 1] - off[e]
        else:
            e, m0, base, M = 0, tile * BM, 0, T
        assert m0 < M and 0 <= e < ne
        rows = min(M - m0, BM)
        NL = 1 if M - m0 <= 32 else 2
        assert 1 <= NL <= MF and 32 * NL >= rows
        # A staging: chunk i = row 32 i + tid / 8, 16-byte chunk tid % 8
        for i in range(NL):
            r = 32 * i + (tid >> 3)
            live = m0 + r < M
            s_ = base + m0 + np.minimum(r, M - m0 - 1)
            assert (s_ < slots).all() and (s_ >= base).all()
            src = xmap[s_] if (mode == 0 and tiles) else s_
            assert (src < arows).all()
            aoff = np.where(live, (src * K + 8 * (tid & 7)) * 2, 0x80000000)
            for t in (0, nkt - 1, nkt + 2):  # the clamped refills past the end repeat the last tile
                k0 = min(t, nkt - 1) * BK
                o = aoff + 2 * k0
                assert ((o[live] + 16) <= bound).all()  # live rows inside A
                assert (o[~live] >= bound).all()       # dead rows past the bound: zeros, no access
                assert (o < 2**31 + 2 * K).all()
            st = r * LD + 8 * (tid & 7)
            assert (st + 8 <= STAGE).all()
        # A fragment reads: row 32 mf + lr, halves 32 h + 8 s .. + 7 of the stage
        for mf in range(NL):
            for s in range(4):
                rd = (32 * mf + lr) * LD + 32 * h + 8 * s
                assert (rd + 8 <= STAGE).all() and ((32 * h + 8 * s + 8) <= BK).all()
        # weight rows of this lane; columns k0 + 32 h .. + 31 (one span), halves 0 and 1 of it
        if mode == 0:
            f = ntile * 128 + 32 * w + lr
            r0 = r1 = f
            assert (f < N).all()
        else:
            r0 = ntile * 256 + 64 * w + lr
            r1 = r0 + 32
            assert (r1 < N).all()
        for k0 in (0, (nkt - 1) * BK):
            c0 = k0 + 32 * h
            assert (c0 % 32 == 0).all() and (c0 + 32 <= K).all()
        # epilogue
        for mf in range(NL):
            for ii in range(16):
                row = 32 * mf + 8 * (ii >> 2) + 4 * h + (ii & 3)
                ok = m0 + row < M
                s = base + m0 + row
                assert (s[ok] < slots).all()
                if mode == 0:
                    col = ntile * 128 + 32 * w + lr
                    np.add.at(written, (s[ok], col[ok]), 1)
                else:
                    for bb in range(2):
                        col = ntile * 256 + 64 * w + 32 * bb + lr
                        np.add.at(written, (s[ok], col[ok]), 1)
    assert (seen == 1).all()  # every (tile, weight-row tile) exactly once
    # mode 0 writes N features of every slot; mode 1 all N rows
    assert (written == 1).all(), (written.min(), written.max())
    return nblk


@pytest.mark.parametrize("args", [
    dict(ne=128, T=2048, nk=8, K=2048, N=768, mode=0), dict(ne=128, T=2048, nk=8, K=768, N=2048, mode=1),
    dict(ne=128, T=64, nk=8, K=2048, N=768, mode=0, skew=1.1), dict(ne=128, T=64, nk=8, K=768, N=2048, mode=1, skew=1.1),
    dict(ne=256, T=8, nk=8, K=2048, N=512, mode=0), dict(ne=512, T=513, nk=10, K=512, N=2048, mode=1, skew=1.1),
    dict(ne=512, T=513, nk=10, K=2048, N=512, mode=0, skew=1.1),
    dict(ne=40, T=300, nk=8, K=4096, N=512, mode=0, skew=1.1),
    dict(ne=1, T=2048, nk=1, K=2048, N=512, mode=0, tiles=False), dict(ne=1, T=200, nk=1, K=512, N=2048, mode=1, tiles=False),
    dict(ne=1, T=161, nk=1, K=1536, N=256, mode=1, tiles=False),
])
def test_gemm_indices_in_range(args):
    assert check(**args) > 0


# packed tiles (k_pack, PkB<F>::ld, the packed branch of gemm3_body): tile bytes and plane offsets
PK_TB = {"Q8_0": 2176, "Q4_K": 1280, "Q5_K": 2304, "Q6_K": 1792}
PK_READS = {  # (offset of lane l's piece, its bytes) in a tile
    "Q8_0": [(lambda l: 16 * l, 16), (lambda l: 1024 + 16 * l, 16), (lambda l: 2048 + 2 * l, 2)],
    "Q4_K": [(lambda l: 16 * l, 16), (lambda l: 1024 + 4 * l, 4)],
    "Q5_K": [(lambda l: 16 * l, 16), (lambda l: 1024 + 16 * l, 16), (lambda l: 2048 + 4 * l, 4)],
    "Q6_K": [(lambda l: 16 * l, 16), (lambda l: 1024 + 8 * l, 8), (lambda l: 1536 + 4 * l, 4)],
}


@pytest.mark.parametrize("fm", sorted(PK_TB))
def test_packed_tile_pieces(fm):
    l = np.arange(64)
    cover = np.zeros(PK_TB[fm], np.int32)
    for off, n in PK_READS[fm]:
        o = off(l)
        assert o.min() >= 0 and (o + n).max() <= PK_TB[fm]
        for x in o:
            cover[x:x + n] += 1
    assert (cover <= 1).all()           # pieces never overlap
    assert (cover == 1).all()           # and fill the tile (no stale bytes between them)


@pytest.mark.parametrize("fm,R,K,ne", [("Q8_0", 768, 2048, 128), ("Q8_0", 2048, 768, 128), ("Q4_K", 512, 2048, 256),
                                       ("Q6_K", 2048, 512, 512), ("Q5_K", 256, 2048, 64), ("Q6_K", 4096, 256, 1)])
def test_pack_and_packed_reads(fm, R, K, ne):
    TB, nkt, ng = PK_TB[fm], K // 64, R // 32
    tiles = ng * nkt
    total = ne * tiles * TB
    l = np.arange(64)
    h, r = l >> 5, l & 31
    # k_pack: grid (tiles, ne), one wave a tile
    for tix in range(tiles):
        g, t = tix // nkt, tix % nkt
        assert (32 * g + r < R).all() and (64 * t + 32 * h + 32 <= K).all()
    assert (ne - 1) * tiles * TB + (tiles - 1) * TB + TB <= total
    # the GEMM's reads: mode 0 (R = ef rows, 128 a block) and mode 1 (R = dm rows, 256 a block)
    for mode, nf in ((0, 128), (1, 256)):
        if R % nf:
            continue
        for ntile in range(R // nf):
            for w in range(4):
                g0 = 4 * ntile + w if mode == 0 else 8 * ntile + 2 * w
                for g in ((g0,) if mode == 0 else (g0, g0 + 1)):
                    assert g < ng
                    for t in (0, nkt - 1):
                        base = (ne - 1) * tiles * TB + (g * nkt + t) * TB
                        for off, n in PK_READS[fm]:
                            assert (base + off(l) + n).max() <= total


# the tile list read off the slot offsets (tiles_load / tiles_total / tiles_find in k_moe_gemm3): lane L of a
# wave holds the tile counts of experts 64 c + L, c < 16; the total is a wave sum; tile i is found by an
# inclusive scan of each chunk and the first lane whose running count passes i
NEC = 16


def tiles_emulated(off, ne):
    assert ne <= 64 * NEC and len(off) == ne + 1
    L = np.arange(64)
    te = np.zeros((NEC, 64), np.int64)
    for c in range(NEC):
        e = 64 * c + L
        ok = e < ne
        te[c, ok] = (off[e[ok] + 1] - off[e[ok]] + BM - 1) // BM
    total = int(sum(te[c].sum() for c in range(NEC) if 64 * c < ne))

    def find(tile):
        acc = 0
        for c in range(NEC):
            if 64 * c >= ne:
                break
            inc = np.cumsum(te[c])
            tot = int(inc[63])
            if tile < acc + tot:
                f = int(np.flatnonzero(acc + inc > tile)[0])
                return 64 * c + f, tile - acc - int(inc[f] - te[c, f])
            acc += tot
        raise AssertionError("tile past the total")
    return total, find


@pytest.mark.parametrize("ne,n,seed,skew", [(128, 512, 0, 1.1), (128, 16384, 1, None), (512, 5130, 2, 1.1),
                                           (1024, 8192, 3, 1.1), (1, 300, 4, None), (65, 64, 5, None),
                                           (1000, 10, 6, None), (200, 0, 7, None)])
def test_tiles_from_offsets(ne, n, seed, skew):
    rng = np.random.default_rng(seed)
    p = np.ones(ne) if skew is None else 1.0 / np.arange(1, ne + 1) ** skew
    ids = rng.choice(ne, n, p=p / p.sum()) if n else np.zeros(0, np.int64)
    cnt = np.bincount(ids, minlength=ne)
    off = np.concatenate([[0], np.cumsum(cnt)])
    tl = [(e, k) for e in range(ne) for k in range((cnt[e] + BM - 1) // BM)]
    total, find = tiles_emulated(off, ne)
    assert total == len(tl) and total <= n // BM + ne + 1   # the grid's bound
    for i, (e, k) in enumerate(tl):
        assert find(i) == (e, k)
        assert 0 <= k * BM < cnt[e]                         # a live slot tile: m0 < M
