"""The grouped GEMM's index arithmetic (k_moe_gemm2 in eureka-engine_amd/csrc/moe_gemm.hip), restated on
the host and run over every block, thread and k-tile of real tile lists: every global read stays inside
its buffer (activation rows past an expert's slots carry an offset past A's buffer bound, which the
buffer load answers with zeros and no access), every LDS access inside its stage, every store inside
the output. Shapes: the 2048-token prefill, Zipf-skewed 64-token batches, and the shared expert.
A change to the kernel's addressing must be mirrored here.
"""
import pytest

import numpy as np  # noqa: E402
BM, BK, LD, BN = 256, 64, 72, 128
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
        maxt = n // BM + ne + 1
        assert len(tl) <= maxt, (len(tl), maxt)
        xmap = np.arange(n) // nk  # slot -> token (any map into [0, T))
        arows = T if mode == 0 else n
    else:
        maxt = (T + BM - 1) // BM
        tl = None
        arows = T
    NF = 64 if mode == 0 else 128
    NT = N // NF
    nblk = 8 * NT * ((maxt + 7) // 8)
    tid = np.arange(512)
    w, l = tid >> 6, tid & 63
    wm, wn = w >> 1, w & 1
    for b in range(nblk):
        bi = b >> 3
        tile = 8 * (bi // NT) + (b & 7)
        ntile = bi % NT
        if tiles:
            if tile >= len(tl): continue
            e, k = tl[tile]
            m0, base, M = k * BM, off[e], off[e + 1] - off[e]
        else:
            e, m0, base, M = 0, tile * BM, 0, T
            if m0 >= M: continue
        assert m0 < M and 0 <= e < ne
        n0 = ntile * NF
        for i in range(4):
            c = tid + 512 * i
            r = c >> 3
            live = m0 + r < M
            s_ = base + m0 + np.minimum(r, M - m0 - 1)
            assert (s_ < (n if tiles else T)).all() and (s_ >= base).all()
            src = (xmap[s_] if (mode == 0 and tiles) else s_)
            assert (src < arows).all()
            bound = arows * K * 2
            aoff = np.where(live, (src * K + 8 * (c & 7)) * 2, 0x80000000)
            for k0 in (0, K - BK):
                o = aoff + 2 * k0
                assert ((o[live] + 16) <= bound).all()           # live rows inside A
                assert (o[~live] >= bound).all()                  # dead rows past the bound: zeros, no access
                assert (o < 2**31 + 2 * K).all() and bound < 2**31
            assert ((r * LD + 8 * (c & 7) + 8) <= BM * LD).all()
        br, bs, bj = tid >> 2, (tid >> 1) & 1, tid & 1
        rowidx = n0 + np.where(br < 64, br, br - 64) if mode == 0 else n0 + br
        assert (rowidx < N).all()
        assert ((K - BK) + 32 * bs + 16 * bj + 16 <= K).all()  # the half-span's columns
        assert (br * LD + 32 * bs + 16 * bj + 16 <= BN * LD).all()
        bro0 = 32 * wn if mode == 0 else 64 * wn
        bro1 = 64 + 32 * wn if mode == 0 else 64 * wn + 32
        assert (64 * wm + 32 + 31 < BM).all() and (bro1 + 31 < BN).all() and (bro0 + 31 < BN).all()
        for a in range(2):
            for ii in range(16):
                row = 64 * wm + 32 * a + 8 * (ii >> 2) + 4 * (l >> 5) + (ii & 3)
                ok = m0 + row < M
                s = base + m0 + row
                assert (s[ok] < (n if tiles else T)).all()
                col = n0 + 32 * wn + (l & 31) if mode == 0 else n0 + 64 * wn + 32 + (l & 31)
                assert (col < N).all()
    return nblk


@pytest.mark.parametrize("args", [
    dict(ne=128, T=2048, nk=8, K=2048, N=768, mode=0), dict(ne=128, T=2048, nk=8, K=768, N=2048, mode=1),
    dict(ne=128, T=64, nk=8, K=2048, N=768, mode=0, skew=1.1), dict(ne=128, T=64, nk=8, K=768, N=2048, mode=1, skew=1.1),
    dict(ne=256, T=8, nk=8, K=2048, N=512, mode=0), dict(ne=512, T=513, nk=10, K=512, N=2048, mode=1, skew=1.1),
    dict(ne=1, T=2048, nk=1, K=2048, N=512, mode=0, tiles=False), dict(ne=1, T=200, nk=1, K=512, N=2048, mode=1, tiles=False),
])
def test_gemm_indices_in_range(args):
    assert check(**args) > 0
