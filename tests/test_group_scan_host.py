"""The dispatch permutation's histogram + scan pair (k_group_count / k_group_place in
eureka-engine_amd/csrc/moe_q8.hip) restated on the host step for step -- blocks of 1024 slots, four waves of
four 64-lane rounds, the per-round ballot passes (leader = the lowest lane left, rank = lanes below with the
same expert + the wave's running count), the per-wave exclusive prefixes, the per-block counts, the scan over
blocks and experts, the placement -- and checked against the oracle's mo_group (pinned to a stable sort in
test_oracle.py) on uniform, Zipf-skewed, single-expert, ragged and one-slot inputs, with every LDS, count and
output index inside its buffer and every position written once. A change to the kernels must be mirrored
here."""
import numpy as np
import pytest

import oracle_lib as ol

GS = 1024


def emulate(ids, nk, ne, rank_above=False):
    n = ids.size
    nb = (n + GS - 1) // GS
    cnt = np.full(nb * ne, 0xDEADBEEF, np.uint64)  # every entry must be written before it is read
    inv = np.full(n, 0xFFFFFFFF, np.uint64)
    passes = 0
    for b in range(nb):
        wc = np.zeros(4 * ne, np.int64)
        rk, ev = {}, {}
        for w in range(4):
            s0 = b * GS + w * 256
            for r in range(4):
                i = s0 + 64 * r + np.arange(64)
                e = np.where(i < n, ids[np.minimum(i, n - 1)], 0xFFFFFFFF).astype(np.int64)
                ok = e < ne
                act = ok.copy()
                my = np.zeros(64, np.int64)
                while act.any():
                    ld = int(np.argmax(act))
                    ee = int(e[ld])
                    same = ok & (e == ee)
                    assert 0 <= w * ne + ee < 4 * ne
                    base = wc[w * ne + ee]
                    below = np.cumsum(same) - same  # lanes under each lane with the same expert
                    if rank_above:  # the mutation control: lanes above instead
                        below = same.sum() - np.cumsum(same)
                    my[same] = base + below[same]
                    wc[w * ne + ee] = base + same.sum()
                    act &= ~same
                    passes += 1
                for L in range(64):
                    rk[(w, r, L)] = my[L]
                    ev[(w, r, L)] = int(e[L]) if ok[L] else None
        pre = np.zeros(4 * ne, np.int64)
        for e in range(ne):
            a = [wc[k * ne + e] for k in range(4)]
            pre[e], pre[ne + e], pre[2 * ne + e], pre[3 * ne + e] = 0, a[0], a[0] + a[1], a[0] + a[1] + a[2]
            cnt[b * ne + e] = sum(a)
        for w in range(4):
            for r in range(4):
                for L in range(64):
                    i = b * GS + w * 256 + 64 * r + L
                    if ev[(w, r, L)] is not None:
                        assert i < n
                        inv[i] = pre[w * ne + ev[(w, r, L)]] + rk[(w, r, L)]
    assert not (cnt == 0xDEADBEEF).any()
    off = np.zeros(ne + 1, np.uint64)
    xmap = np.full(n, 0xFFFFFFFF, np.uint64)
    written = np.zeros(n, np.int32)
    inv2 = inv.copy()
    for b in range(nb):
        # thread t: experts 4 t .. 4 t + 3; the exclusive scan over threads in expert order
        tot = np.array([cnt[k * ne:(k + 1) * ne] for k in range(nb)]).sum(0)
        bef = np.array([cnt[k * ne:(k + 1) * ne] for k in range(b)]).sum(0) if b else np.zeros(ne, np.uint64)
        assert ne <= 1024
        pre_e = np.concatenate([[0], np.cumsum(tot)[:-1]])
        base = pre_e + bef
        if b == 0:
            off[:ne] = pre_e
            off[ne] = n
        for q in range(4):
            for t in range(256):
                i = b * GS + 256 * q + t
                if i < n and ids[i] < ne:
                    pos = int(base[ids[i]] + inv[i])
                    assert 0 <= pos < n
                    inv2[i] = pos
                    xmap[pos] = i // nk
                    written[pos] += 1
    assert (written[:int(off[ne])] <= 1).all()
    return off.astype(np.uint32), xmap, inv2, passes


def _oracle(ids, nk, ne):
    n = ids.size
    ro, rx, rv = np.zeros(ne + 1, np.uint32), np.zeros(n, np.uint32), np.zeros(n, np.uint32)
    ids = np.ascontiguousarray(ids, np.uint32)
    ol.lib().mo_group(ol.ptr(ids), n, nk, ne, ol.ptr(ro), ol.ptr(rx), ol.ptr(rv))
    return ro, rx, rv


def _zipf_ids(T, nk, ne, seed):
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, ne + 1) ** 1.1
    p = p[rng.permutation(ne)]
    p /= p.sum()
    return np.stack([rng.choice(ne, nk, replace=False, p=p) for _ in range(T)]).ravel().astype(np.uint32)


CASES = {
    "uniform_c4": lambda: (np.stack([np.random.default_rng(1).permutation(128)[:8] for _ in range(300)]).ravel(), 8, 128),
    "zipf_c3": lambda: (_zipf_ids(64, 8, 128, 3), 8, 128),
    "zipf_c5": lambda: (_zipf_ids(513, 10, 512, 5), 10, 512),
    "one_expert_spans_blocks": lambda: (np.zeros(2500, np.uint32), 1, 4),
    "ragged_tail": lambda: (np.random.default_rng(7).integers(0, 1000, 1027 * 3).astype(np.uint32), 3, 1000),
    "one_slot": lambda: (np.array([5], np.uint32), 1, 8),
    "ne_1024": lambda: (np.random.default_rng(9).integers(0, 1024, 4096).astype(np.uint32), 4, 1024),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_group_scan_emulation_matches_the_oracle(case):
    ids, nk, ne = CASES[case]()
    ids = np.asarray(ids, np.uint32)
    o, x, v, passes = emulate(ids, nk, ne)
    ro, rx, rv = _oracle(ids, nk, ne)
    assert np.array_equal(o, ro)
    assert np.array_equal(x.astype(np.uint32), rx) and np.array_equal(v.astype(np.uint32), rv)
    nrounds = 16 * ((ids.size + GS - 1) // GS)
    assert passes <= 64 * nrounds


def test_group_scan_emulation_control():
    """mutation control: ranking a round's lanes by the lanes above (not below) gives another permutation"""
    ids, nk, ne = CASES["zipf_c3"]()
    _, x, _, _ = emulate(np.asarray(ids, np.uint32), nk, ne, rank_above=True)
    _, rx, _ = _oracle(ids, nk, ne)
    assert not np.array_equal(x.astype(np.uint32), rx)
