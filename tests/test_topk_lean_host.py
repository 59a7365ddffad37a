"""The one-token decode's lean top-k (topk_block4 in eureka-engine_amd/csrc/moe_decode.hip, selected by
llb_moe_hip_set_lean_topk) restated on the host step for step: the max and the 32-expert group sums, the
64-bit keys (p bits + 1, then the inverted index), each key's place in its 64-expert group counted against
the group's 64 keys, the first nc = min(nk, 16) places as candidates (key 0 elsewhere), each candidate's rank
among the 64 candidate slots, the slots named by ranks below nk with a real p, then the rank-order
renormalisation. Checked bit for bit against the oracle's mo_topk (pinned in test_oracle.py) on the tie
patterns of the GPU routing test, NaN and -inf logits, ne 1..256 and nk 1..16. A change to the kernel must
be mirrored here."""
import numpy as np
import pytest

import oracle_lib as ol

F = np.float32


def emulate(lg, ne, nk, rank_place_only=False):
    lg = np.asarray(lg, F)
    t = np.arange(256)
    v = np.where(t < ne, np.concatenate([lg, np.zeros(256 - ne, F)]), F(0))
    with np.errstate(invalid="ignore"):
        vm = np.where(t < ne, v, F(-np.inf)).astype(F)
    # wave_fmax: fmaxf tree (NaN-ignoring) over the wave's lanes
    red = []
    for w in range(4):
        x = vm[64 * w:64 * w + 64]
        m = F(-np.inf)
        for a in x:
            m = F(np.fmax(m, a))
        red.append(m)
    mx = red[0]
    for i in range(1, 4):
        mx = F(np.fmax(mx, red[i]))
    with np.errstate(all="ignore"):
        ev = np.where(t < ne, np.array([F(np.exp(np.float64(F(a - mx)))) for a in v], F), F(0)).astype(F)
    # group sums: xor butterfly 16, 8, 4, 2, 1 over each 32-lane group (lane 0's value)
    gs = []
    for g in range(8):
        a = ev[32 * g:32 * g + 32].copy()
        for m in (16, 8, 4, 2, 1):
            a = np.array([F(a[i] + a[i ^ m]) for i in range(32)], F)
        gs.append(a[0])
    tot = F(0)
    for g in range(8):
        tot = F(tot + gs[g])
    inv = F(F(1) / tot)
    with np.errstate(invalid="ignore"):
        p = (ev * inv).astype(F)
    kb = np.where((t < ne) & (p >= 0), p.view(np.uint32).astype(np.uint64) + 1, 0).astype(np.uint64)
    key = (kb << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - t.astype(np.uint64))
    nc = min(nk, 16)
    cand = np.zeros(64, np.uint64)
    for w in range(4):
        k = key[64 * w:64 * w + 64]
        place = np.array([(k > k[L]).sum() for L in range(64)])
        for L in range(64):
            if place[L] < nc:
                cand[16 * w + place[L]] = k[L]
    sid, sp = np.zeros(64, np.uint32), np.zeros(64, F)
    for i in range(64):
        if i % 16 >= nc:
            continue
        rk = int((cand > cand[i]).sum())
        if rank_place_only:
            rk = i % 16  # mutation control: a candidate's place in its group taken as its rank
        mh = int(cand[i] >> np.uint64(32))
        if rk < nk and mh != 0:
            sid[rk] = 0xFFFFFFFF - int(cand[i] & np.uint64(0xFFFFFFFF))
            sp[rk] = np.uint32(mh - 1).view(F)
    s = F(0)
    for j in range(nk):
        s = F(s + sp[j])
    s = s if s >= F(6.103515625e-5) else F(6.103515625e-5)
    wt = (sp[:nk] / s).astype(F)
    return sid[:nk], wt


def _oracle(lg, ne, nk):
    ids, wt, sgo = np.zeros(nk, np.uint32), np.zeros(nk, F), np.zeros(1, F)
    lgc = np.ascontiguousarray(lg, F)
    ol.lib().mo_topk(ol.ptr(lgc), ne, nk, 0.0, ol.ptr(ids), ol.ptr(wt), ol.ptr(sgo))
    return ids, wt


def _rows(ne, nk, rng):
    rows = [rng.standard_normal(ne), np.round(rng.standard_normal(ne) * 2) / 2, np.zeros(ne)]
    for ntop in (64, 65):
        r = rng.standard_normal(ne) - 10.0
        r[rng.permutation(ne)[:min(ntop, ne)]] = 3.0
        rows.append(r)
    r = np.sort(rng.standard_normal(ne))[::-1].copy()
    if nk < ne:
        r[nk - 1] = r[nk]
    rows.append(rng.permutation(r))
    r = np.zeros(ne)
    r[ne // 2] = 5.0
    rows.append(r)
    r = rng.standard_normal(ne)
    r[rng.permutation(ne)[:3]] = -np.inf
    rows.append(r)
    r = rng.standard_normal(ne)
    r[0] = np.nan
    rows.append(r)
    return [np.asarray(x, F) for x in rows]


@pytest.mark.parametrize("ne,nk", [(256, 8), (128, 8), (200, 16), (64, 1), (130, 15), (1, 1), (256, 16), (65, 3)])
def test_lean_topk_emulation_matches_the_oracle(ne, nk):
    rng = np.random.default_rng(ne * 100 + nk)
    for i, lg in enumerate(_rows(ne, nk, rng)):
        gi, gw = emulate(lg, ne, nk)
        ri, rw = _oracle(lg, ne, nk)
        assert np.array_equal(gi, ri), (i, gi, ri)
        assert np.array_equal(gw.view(np.uint32), rw.view(np.uint32)), i


def test_lean_topk_control():
    """mutation control: taking a candidate's place in its group for its rank fails"""
    rng = np.random.default_rng(3)
    lg = rng.standard_normal(256).astype(F)
    gi, _ = emulate(lg, 256, 8, rank_place_only=True)
    ri, _ = _oracle(lg, 256, 8)
    assert not np.array_equal(gi, ri)
