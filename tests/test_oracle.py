"""CPU checks that pin the oracle (oracle/moe_oracle.c) before it is trusted as the GPU's checker.

Each check is independent of the oracle's own code: the reference's compiled C (oracle/_ref, built
from tools/qwen35_engine.c), numpy, hand-derived known answers that tell the dot orders apart,
brute force, and a float64 recompute with mutation controls that must fail.
"""
import ctypes as C

import numpy as np
import pytest

import eureka_moe as em
import oracle_lib as ol

lib = ol.lib()


def f32(x):
    return np.float32(x)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def nan_eq(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return bool(np.all((np.isnan(a) & np.isnan(b)) | (bits(a) == bits(b))))


# ---------------------------------------------------------------- f16

def test_f16_exhaustive_against_numpy_and_reference():
    h = np.arange(65536, dtype=np.uint32)
    mine = np.array([lib.mo_f16(int(v)) for v in h], np.float32)
    npy = h.astype(np.uint16).view(np.float16).astype(np.float32)
    assert nan_eq(mine, npy)
    # (NaN payloads are compared array to array through mo_deq_row in the dequant tests: a float
    # returned through ctypes passes a double conversion that quiets a signalling NaN)
    ref = ol.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    rv = np.array([ref.ref_half_to_float(int(v)) for v in h], np.float32)
    assert nan_eq(mine, rv)


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
                        np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, -6.0e-8, 5.96e-8, np.inf, -np.inf])]).astype(np.float32)
    mine = np.array([lib.mo_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(mine, x.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------- dequant

def _ref_deq(fm, row, cols):
    out = np.zeros(cols, np.float32)
    ol.ref_lib().ref_deq_row(fm, ol.ptr(row), cols, ol.ptr(out))
    return out


@pytest.mark.parametrize("fm", [em.Q4_K, em.Q6_K, em.Q5_K])
def test_kquant_dequant_matches_reference_build(fm):
    if ol.ref_lib() is None:
        pytest.skip("oracle/_ref not built")
    rng = np.random.default_rng(fm)
    cols = 1024
    for trial in range(40):
        row = rng.integers(0, 256, em.row_bytes(fm, cols), dtype=np.uint8)
        if trial % 4 == 0:  # keep the f16 scales finite and small so the values are ordinary
            bb = em.BLOCK[fm][0]
            for b in range(cols // 256):
                o = b * bb + (208 if fm == em.Q6_K else 0)
                row[o:o + 2] = np.frombuffer(np.float16(rng.uniform(-1, 1)).tobytes(), np.uint8)
        assert nan_eq(ol.deq(fm, row, cols), _ref_deq(fm, row, cols))


def test_q8_0_gguf_blocks_match_reference_row_split():
    """the expert stacks keep GGUF Q8_0 blocks ([d][32 q]); the reference CPU twin reads the trunk's
    row split ([q x cols][d x cols/32], tools/q8_pack.py): the same values after re-laying the bytes"""
    if ol.ref_lib() is None:
        pytest.skip("oracle/_ref not built")
    rng = np.random.default_rng(8)
    cols = 768
    blocks = rng.integers(0, 256, (cols // 32, 34), dtype=np.uint8)
    split = np.concatenate([blocks[:, 2:].ravel(), blocks[:, :2].ravel()])
    assert nan_eq(ol.deq(em.Q8_0, blocks.ravel().copy(), cols), _ref_deq(em.Q8_0, split, cols))


def test_dequant_known_answers():
    # Q4_K: d = 1, dmin = 0.5, sub-block 0 scale 3 min 2, first nibble 5 -> 1 * 3 * 5 - 0.5 * 2 = 14
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[4] = 3   # scale of sub-block 0 (low 6 bits)
    blk[8] = 2   # min of sub-block 0
    blk[16] = 0x75  # col 0 nibble 5, col 32 nibble 7 (sub-block 1: scale 0, min 0 -> 0)
    w = ol.deq(em.Q4_K, blk, 256)
    assert w[0] == 14.0 and w[32] == 0.0 and w[1] == -1.0
    # sub-block 4 takes its scale's high bits from byte 4 + 0 (get_scale_min_k4): sc = (b[8] & 15) | (b[0] >> 6) << 4
    blk2 = np.zeros(144, np.uint8)
    blk2[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk2[4] = 0b11000000   # sub-block 0 scale 0, high bits 3 for sub-block 4
    blk2[12] = 0b00000101  # low nibble 5 of sub-block 4's scale
    blk2[16 + 64] = 0x01   # col 128 (sub-block 4) nibble 1
    assert ol.deq(em.Q4_K, blk2, 256)[128] == float((3 << 4) | 5)
    # Q6_K: q = 0 -> -32 * d * sc; q = 63 -> 31 * d * sc
    b6 = np.zeros(210, np.uint8)
    b6[208:210] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    b6[192] = 4                      # scale of cols 0..15
    b6[0] = 0x0F                     # col 0 low nibble 15
    b6[128] = 0x03                   # col 0 high bits 3 -> q = 63
    w6 = ol.deq(em.Q6_K, b6, 256)
    assert w6[0] == 31.0 and w6[1] == -32.0 and w6[16] == -0.0
    # Q8_0: q * d, signed
    b8 = np.zeros(34, np.uint8)
    b8[0:2] = np.frombuffer(np.float16(-2.0).tobytes(), np.uint8)
    b8[2], b8[3] = 3, 0xFD
    w8 = ol.deq(em.Q8_0, b8, 32)
    assert w8[0] == -6.0 and w8[1] == 6.0 and bits(w8[2]) == 0x80000000  # 0 * -2 = -0


# ---------------------------------------------------------------- dot orders (known answers)

def _f32_row(groups, cols=2048):
    """a row whose group g leaf is groups[g] (w = [v, 0, 0, 0], x = 1)"""
    w = np.zeros(cols, np.float32)
    for g, v in groups.items():
        w[4 * g] = v
    return w, np.ones(cols, np.float32)


BIG = float(2 ** 24)


def test_tree_order_known_answer():
    # leaves 0: 2^24, 2: 1, 3: 1. The tree adds (2 + 3) = 2 before it meets 2^24: 2^24 + 2 is exact.
    # Strided lanes add 2^24 + 1 (lane 2 into lane 0 at level 2) -> 2^24, then + 1 -> 2^24.
    w, x = _f32_row({0: BIG, 2: 1.0, 3: 1.0})
    assert lib.mo_dot_tree(em.F32, ol.ptr(w), 2048, ol.ptr(x)) == BIG + 2
    assert lib.mo_dot_stride(em.F32, ol.ptr(w), 2048, ol.ptr(x)) == BIG
    ref = ol.ref_lib()
    if ref is not None:  # the reference's CPU twin sums in order: 2^24 + 1 + 1 -> 2^24
        assert ref.ref_dot_fmt(0, ol.ptr(w), 2048, ol.ptr(x)) == BIG


def test_stride_order_known_answer():
    # leaves 0: 2^24, 1: 1, 33: 1. Lane 1 of 32 holds groups 1 and 33: 1 + 1 = 2, then 2^24 + 2 exact.
    # The tree meets 2^24 + 1 (groups 0, 1) first -> 2^24, and the right half's 1 rounds away too.
    w, x = _f32_row({0: BIG, 1: 1.0, 33: 1.0})
    assert lib.mo_dot_stride(em.F32, ol.ptr(w), 2048, ol.ptr(x)) == BIG + 2
    assert lib.mo_dot_tree(em.F32, ol.ptr(w), 2048, ol.ptr(x)) == BIG


def test_stride_butterfly_level_order():
    # lanes 0: 2^24, 16: 1, 8: 1, 24: 1 (groups 0, 16, 8, 24). Level 16 pairs (0,16) -> 2^24 and
    # (8,24) -> 2; level 8 adds them: 2^24 + 2. If level 1 came first nothing would pair differently
    # here, but levels 8-before-16 would give (0,8) -> 2^24, (16,24) -> 2: the same. Use lanes
    # 0: 2^24, 16: 1, 24: 1 instead: 16-first gives 2^24 + (1 + 1) = 2^24 + 2; 8-first gives
    # (0 + 8) = 2^24, (16 + 24) = 2 -> 2^24 + 2 as well; and 1-first the same. So also check
    # the leaf: (w0 x0 + w1 x1) + (w2 x2 + w3 x3) with 2^24, 1, 1, 0 in one group -> 2^24 + 1 = 2^24, + 1
    w = np.zeros(2048, np.float32)
    x = np.ones(2048, np.float32)
    w[0], w[2], w[3] = BIG, 1.0, 1.0  # leaf 0 = (2^24 + 0) + (1 + 1) = 2^24 + 2
    assert lib.mo_dot_stride(em.F32, ol.ptr(w), 2048, ol.ptr(x)) == BIG + 2
    w[0], w[1], w[2], w[3] = BIG, 1.0, 1.0, 0.0  # (2^24 + 1) + (1 + 0) -> 2^24 + 1 -> 2^24
    assert lib.mo_dot_stride(em.F32, ol.ptr(w), 2048, ol.ptr(x)) == BIG


@pytest.mark.parametrize("fm,cols", [(em.F32, 2048), (em.Q4_K, 2048), (em.Q6_K, 512), (em.Q8_0, 768), (em.Q5_K, 1024)])
def test_dots_close_to_float64(fm, cols):
    rng = np.random.default_rng(cols + fm)
    row = ol.gen_rows(fm, 3, 1, 0, 1, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    w = ol.deq(fm, row, cols).astype(np.float64)
    exact = float(w @ x)
    scale = float(np.abs(w) @ np.abs(x))
    for f in (lib.mo_dot_stride, lib.mo_dot_tree):
        assert abs(f(fm, ol.ptr(row), cols, ol.ptr(x)) - exact) <= 1e-6 * scale


def test_tuned_predicate_follows_llb_tuned():
    # llb_tuned (host/llb_host.c:64-76): F32 at cdepth 9..12; K-quants whole quads 8..13 or 9..11
    assert lib.mo_cdepth(2048) == 9 and lib.mo_cdepth(512) == 7 and lib.mo_cdepth(1025) == 9
    assert lib.mo_tuned(em.F32, 2048) and not lib.mo_tuned(em.F32, 1024)
    assert lib.mo_tuned(em.Q4_K, 2048) and lib.mo_tuned(em.Q4_K, 1024)
    assert not lib.mo_tuned(em.Q6_K, 512) and lib.mo_tuned(em.Q6_K, 1536)
    assert not lib.mo_tuned(em.Q5_K, 1536) and lib.mo_tuned(em.Q5_K, 1024)


# ---------------------------------------------------------------- routing and permutation

def _topk(lg, nk, sg=0.0):
    ne = lg.size
    ids, wt, sgo = np.zeros(nk, np.uint32), np.zeros(nk, np.float32), np.zeros(1, np.float32)
    lgc = np.ascontiguousarray(lg, np.float32)  # held while the oracle reads it
    lib.mo_topk(ol.ptr(lgc), ne, nk, float(sg), ol.ptr(ids), ol.ptr(wt), ol.ptr(sgo))
    return ids, wt, sgo[0]


@pytest.mark.parametrize("ne,nk", [(128, 8), (256, 8), (512, 10), (8, 8), (1, 1), (2000, 6)])
def test_topk_against_float64_sort(ne, nk):
    rng = np.random.default_rng(ne)
    lg = (rng.permutation(ne).astype(np.float64) * 0.01).astype(np.float32)  # distinct, well separated
    ids, wt, sgo = _topk(lg, nk, sg=0.3)
    p = np.exp(lg.astype(np.float64) - lg.max())
    p /= p.sum()
    want = np.argsort(-p, kind="stable")[:nk]
    assert list(ids) == list(want)
    w64 = p[want] / p[want].sum()
    assert np.allclose(wt, w64, rtol=2e-6, atol=1e-7)
    assert abs(float(wt.astype(np.float64).sum()) - 1.0) <= nk * 2 ** -23
    assert abs(sgo - 1 / (1 + np.exp(-0.3))) < 1e-7
    assert np.all(np.diff(wt) <= 0) and len(set(ids.tolist())) == nk


def test_topk_ties_go_to_the_lower_index():
    ids, wt, _ = _topk(np.zeros(64, np.float32), 5)
    assert list(ids) == [0, 1, 2, 3, 4] and np.all(wt == np.float32(0.2))
    lg = np.array([1, 3, 3, 0, 3, 2], np.float32)
    assert list(_topk(lg, 4)[0]) == [1, 2, 4, 5]


def test_topk_full_softmax_when_k_is_ne():
    lg = np.array([0.5, -1.0, 2.0, 0.0], np.float32)
    ids, wt, _ = _topk(lg, 4)
    p = np.exp(lg.astype(np.float64) - 2.0)
    p /= p.sum()
    assert list(ids) == [2, 0, 3, 1]
    assert np.allclose(wt, p[[2, 0, 3, 1]], rtol=1e-6)


def test_group_is_a_stable_sort():
    rng = np.random.default_rng(5)
    for T, nk, ne in [(1, 8, 256), (64, 8, 128), (300, 10, 512), (7, 3, 4)]:
        ids = np.stack([rng.permutation(ne)[:nk] for _ in range(T)]).astype(np.uint32).ravel()
        n = ids.size
        off, xm, inv = np.zeros(ne + 1, np.uint32), np.zeros(n, np.uint32), np.zeros(n, np.uint32)
        lib.mo_group(ol.ptr(ids), n, nk, ne, ol.ptr(off), ol.ptr(xm), ol.ptr(inv))
        order = np.argsort(ids, kind="stable")
        assert np.array_equal(xm, order // nk)
        assert np.array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(ids, minlength=ne))]))
        assert np.array_equal(order[inv], np.arange(n))  # inv maps each slot to its position


def test_q8_1_against_numpy():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(1024).astype(np.float32)
    x[:32] = 0.0
    q, d, s = np.zeros(1024, np.int8), np.zeros(32, np.float32), np.zeros(32, np.float32)
    lib.mo_q8_1(ol.ptr(x), 1024, ol.ptr(q), ol.ptr(d), ol.ptr(s))
    xb = x.reshape(32, 32)
    dd = (np.abs(xb).max(1) / np.float32(127)).astype(np.float32)
    assert np.array_equal(d, dd)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = xb / dd[:, None]
    qq = np.where(dd[:, None] == 0, 0, np.sign(r) * np.floor(np.abs(r) + 0.5)).astype(np.int8)  # roundf: half away
    assert np.array_equal(q.reshape(32, 32), qq)
    assert np.allclose(s, xb.astype(np.float64).sum(1), atol=1e-4)


# ---------------------------------------------------------------- quantizers and the generator

@pytest.mark.parametrize("fm,tol", [(em.Q8_0, 0.51), (em.Q4_K, 1.01), (em.Q5_K, 1.01), (em.Q6_K, 0.75)])
def test_quantizer_round_trip(fm, tol):
    x = ol.gauss(11, 2, 0, 4096, 0.02)
    row = np.zeros(em.row_bytes(fm, 4096), np.uint8)
    assert lib.mo_quant_row(fm, ol.ptr(x), 4096, ol.ptr(row)) == 0
    w = ol.deq(fm, row, 4096)
    step = {em.Q8_0: x.reshape(-1, 32), em.Q4_K: x.reshape(-1, 32), em.Q5_K: x.reshape(-1, 32),
            em.Q6_K: x.reshape(-1, 16)}[fm]
    levels = {em.Q8_0: 127, em.Q4_K: 7.5, em.Q5_K: 15.5, em.Q6_K: 31}[fm]
    span = np.abs(step).max(1) if fm in (em.Q8_0, em.Q6_K) else (step.max(1) - np.minimum(step.min(1), 0)) / 2
    err = np.abs(w - x).reshape(step.shape).max(1)
    # half a quantization step plus the 6-bit scale code's rounding
    assert np.all(err <= tol * span / levels * 1.1 + 1e-7), float((err / (span / levels)).max())


def test_gauss_moments_and_determinism():
    x = ol.gauss(0, 0, 0, 200000, 1.0).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert np.array_equal(ol.gauss(0, 0, 100, 10), x[100:110].astype(np.float32))
    assert not np.array_equal(ol.gauss(1, 0, 0, 10), x[:10].astype(np.float32))


# ---------------------------------------------------------------- the layer against float64

SMALL = em.Shape(2048, 16, 4, 256, 256, em.Q4_K, em.Q4_K, em.Q6_K)


def test_exact_layer_matches_float64_and_mutants_fail():
    h2, x1 = ol.inputs(SMALL, 3, 2)
    hl = ol.HostLayer(SMALL, seed=3, experts=range(SMALL.ne))
    y, ids, wt, sgo = hl.run(h2, None)
    y64 = hl.f64(h2, ids)
    m = ol.err_metrics(y, y64)
    assert m["rel"] < 1e-5 and m["cos"] > 0.9999999, m
    # the residual adds exactly
    yr, _, _, _ = hl.run(h2, x1)
    assert np.allclose(yr - x1, y, atol=1e-5)
    # mutation controls (reports/cuda-moe/REPORT.md:100-108): each must fail the check
    lowest = np.stack([np.argsort(np.abs(w))[:SMALL.nk] for w in [np.zeros(SMALL.ne)] * 2])
    bad_ids = (ids + 1) % SMALL.ne
    assert ol.err_metrics(y, hl.f64(h2, bad_ids))["rel"] > 0.1
    assert lowest.shape == ids.shape
    no_renorm = y * np.float32(1.3)
    assert ol.err_metrics(no_renorm, y64)["rel"] > 0.05


def test_q8_tier_close_to_exact():
    h2, _ = ol.inputs(SMALL, 4, 2)
    hl = ol.HostLayer(SMALL, seed=4, experts=range(SMALL.ne))
    y, ids, _, _ = hl.run(h2, None)
    yq, idq, _, _ = hl.run(h2, None, tier="q8")
    assert np.array_equal(ids, idq)
    m = ol.err_metrics(yq, y)
    assert m["rel"] < 0.05 and m["cos"] > 0.998, m


def test_oracle_threads_give_the_same_bits():
    h2, _ = ol.inputs(SMALL, 6, 1)
    hl = ol.HostLayer(SMALL, seed=6, experts=range(SMALL.ne))
    y1, _, _, _ = hl.run(h2, None, nthreads=1)
    y4, _, _, _ = hl.run(h2, None, nthreads=4)
    assert np.array_equal(bits(y1), bits(y4))


def _exp_hit(k):
    """a float x whose exp through F64, rounded to float, is exactly 2^-k (the oracle's exp is
    (float)exp((double)x), pinned against the reference's hf_exp above)"""
    x0 = np.float32(-k * np.log(2))
    for d in range(200):
        for s in (1, -1):
            x = x0
            for _ in range(d):
                x = np.nextafter(x, np.float32(100 * s))
            if np.float32(np.exp(np.float64(x))) == np.float32(2.0 ** -k):
                return x
    raise AssertionError(k)


def test_topk_softmax_sum_order_known_answer():
    """llb_moe_topk's sum (tools/payload-moeany.patch:346-371): thread t of 1024 adds p[e], e = t mod 1024,
    in ascending e; each warp of 32 folds by xor 16, 8, 4, 2, 1 (own value first); thread 0 adds the 32
    warp sums in order from 0. The case below has only powers of two, so each partial sum can be followed
    by hand, and the 1024-thread order gives a different total from a sequential sum and from a 256-thread
    block, and through it different weights.

    ne = 16384. p = 1 at e = l + 256 j (l < 32, j < 32: 1024 ones), p = 2^-14 at e = 8224 and 8256,
    p = 1/2 at e = 10241, p = 0 elsewhere (logit -inf).
      sequential: the ones end at e = 7967 with 1024; each 2^-14 then is half an ulp of 1024 and ties to
        even (1024); + 1/2 -> 1024.5.
      256 threads: warp 0 (e mod 256 < 32) holds every one and the 1/2: 1024.5; warps 1 and 2 hold one
        2^-14 each, and each ties away at 1024.5 (its last mantissa bit is even) -> 1024.5.
      1024 threads: thread l + 256 q holds 8 ones; warps 0, 8, 16, 24 sum 256 (warp 0 256.5); warps 1
        and 2 hold the two 2^-14 and meet the total while it is 256.5 (ulp 2^-15): exact. The total runs
        256.5, +2^-14, +2^-14, 512.5 + 2^-13, 768.5 + 2^-13, 1024.5 + 2^-13: exact throughout.
    With k = 3 (ids 0, 1, 2, all p = 1) the weights are inv / (3 inv), inv = 1 / total, renormalised: the
    two totals give different bits."""
    ne, nk = 16384, 3
    lg = np.full(ne, -np.inf, np.float32)
    for l in range(32):
        lg[l + 256 * np.arange(32)] = 0.0
    lg[[8224, 8256]] = _exp_hit(14)
    lg[1 + 256 * 40] = _exp_hit(1)
    ids, wt, _ = _topk(lg, nk)
    assert list(ids) == [0, 1, 2]

    def weights(total):
        inv = np.float32(1.0) / np.float32(total)
        s = np.float32(np.float32(inv + inv) + inv)
        return np.full(nk, inv / s, np.float32)

    want = weights(1024.5 + 2.0 ** -13)
    other = weights(1024.5)  # the sequential and the 256-thread totals
    assert not np.array_equal(want.view(np.uint32), other.view(np.uint32))
    assert np.array_equal(wt.view(np.uint32), want.view(np.uint32))


def _q4dp():
    r = ol.ref_q4dp()
    if r is None:
        pytest.skip("oracle/_ref/libref_q4dp.so is not built (make -C oracle ref; needs the reference tree)")
    return r


def _q8_1(x):
    n = x.size
    q, d, s = np.zeros(n, np.int8), np.zeros(n // 32, np.float32), np.zeros(n // 32, np.float32)
    lib.mo_q8_1(ol.ptr(x), n, ol.ptr(q), ol.ptr(d), ol.ptr(s))
    return q, d, s


def test_q8_1_matches_the_reference_twin():
    """q and d bit for bit against ref_q8x (tools/q4dp/q4dp_ref.h:18-30) on finite blocks: normal, zero,
    tiny (subnormal d), huge, one-hot, and halfway values that roundf takes away from zero. (For a block
    holding inf / NaN the twin stores d = NaN and q = 0; pf_q8x, which the oracle follows, has no such
    branch: such inputs are outside the path's envelope.)"""
    r = _q4dp()
    rng = np.random.default_rng(11)
    x = rng.standard_normal(32 * 64).astype(np.float32)
    xb = x.reshape(64, 32)
    xb[1] = 0.0
    xb[2] *= np.float32(1e-38)
    xb[3] *= np.float32(1e36)
    xb[4] = 0.0
    xb[4, 7] = -3.0
    xb[5] = (np.arange(32, dtype=np.float32) - 16.0) + 0.5  # amax 16.5: x / d lands near halves
    xb[6] = np.float32(127.0) * (np.arange(32) % 3 - 1).astype(np.float32) / np.float32(2.0)
    q, d, _ = _q8_1(x)
    rq, rd = np.zeros(x.size, np.int8), np.zeros(64, np.float32)
    r.ref_q8x_c(ol.ptr(x), ol.ptr(rq), ol.ptr(rd), x.size)
    assert np.array_equal(q, rq)
    assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))


def test_q8_1_sum_is_the_warp_butterfly():
    """s is pf_q8x's xor-butterfly sum (tools/pf27/pfmm.cuh:44-48), lane 0's value. x0 = 2^24, x1 = x3 =
    1: the butterfly meets x1 + x3 = 2 (level 2) before 2^24 (level 1): 2^24 + 2, exact. A sequential
    sum loses each 1 against 2^24: 2^24."""
    x = np.zeros(32, np.float32)
    x[0], x[1], x[3] = BIG, 1.0, 1.0
    _, _, s = _q8_1(x)
    assert s[0] == BIG + 2


def _q4k_exact_case(rng, nsb):
    """a Q4_K row and q8_1 activations on which every product and sum of the block dot is exact in f32:
    d = 2^-8, dmin = 2^-9, each 32-block of x is q dx with |q| <= 3 but one +-127, dx = 2^-6 or 2^-7
    (so d = amax / 127 = dx exactly and x / d = q), scales and nibbles random."""
    row = bytearray()
    for _ in range(nsb):
        row += (0x1C00).to_bytes(2, "little") + (0x1800).to_bytes(2, "little")
        row += bytes(rng.integers(0, 256, 12, dtype=np.uint8)) + bytes(rng.integers(0, 256, 128, dtype=np.uint8))
    cols = 256 * nsb
    q = rng.integers(-3, 4, cols).astype(np.int8).reshape(-1, 32)
    q[np.arange(q.shape[0]), rng.integers(0, 32, q.shape[0])] = np.where(rng.random(q.shape[0]) < 0.5, 127, -127)
    dx = np.where(rng.random(q.shape[0]) < 0.5, 2.0 ** -6, 2.0 ** -7).astype(np.float32)
    x = (q.astype(np.float32) * dx[:, None]).ravel()
    return np.frombuffer(bytes(row), np.uint8).copy(), x


def _q4k_f64(row, x, nsb):
    """the block dot in float64 from the format's definition (d sc q - dmin m per weight, times x)"""
    w = np.zeros(256 * nsb, np.float32)
    lib.mo_deq_row(em.Q4_K, ol.ptr(row), 256 * nsb, ol.ptr(w))
    return float(np.dot(w.astype(np.float64), x.astype(np.float64)))


@pytest.mark.parametrize("nsb", [1, 4])
def test_q4k_block_dot_matches_the_reference_twin_and_its_mutants_fail(nsb):
    """mo_dot_q8's Q4_K block dot (mx_blk, host/llb_pf.cuh:468-515) against the reference's twin ref_row /
    ref_sb (tools/q4dp/q4dp_ref.h:32-74), bit for bit, on rows where all arithmetic is exact (so the two
    summation orders and s = sum x against dx sum q cannot differ), and against float64 from the
    dequantised row. The twin's own mutation controls (mut 1: a scale + 1, 2: nibbles swapped, 3: x one
    block off, 4: the dmin term's sign) must each give another value."""
    r = _q4dp()
    rng = np.random.default_rng(40 + nsb)
    for _ in range(8):
        row, x = _q4k_exact_case(rng, nsb)
        cols = 256 * nsb
        q, d, s = _q8_1(x)
        assert np.array_equal(q.astype(np.float32) * np.repeat(d, 32), x)  # the q8_1 is exact
        ours = lib.mo_dot_q8(em.Q4_K, ol.ptr(row), cols, ol.ptr(q), ol.ptr(d), ol.ptr(s))
        theirs = r.ref_row_c(ol.ptr(row), nsb, ol.ptr(q), ol.ptr(d), cols, 0)
        exact = _q4k_f64(row, x, nsb)
        assert ours == theirs == exact
        shares = sum(float(r.ref_sb_c(ol.ptr(row[144 * sb:]), ol.ptr(q), ol.ptr(d), cols, sb, g, k, 0))
                     for sb in range(nsb) for g in range(4) for k in range(4))
        assert shares == exact
        for mut in (1, 2, 3, 4):
            assert r.ref_row_c(ol.ptr(row), nsb, ol.ptr(q), ol.ptr(d), cols, mut) != ours, mut


def _exact_row(rng, fm, cols):
    """a row of format fm whose every block dot against exact q8_1 activations is exact in f32: f16 scales
    2^-8 / 2^-9 and 6-bit or int8 sub-scales kept small; the quant bits random"""
    nb = cols // 256
    out = bytearray()
    if fm == em.Q8_0:
        for _ in range(cols // 32):
            out += (0x1C00).to_bytes(2, "little") + bytes(rng.integers(0, 256, 32, dtype=np.uint8))
    elif fm == em.Q6_K:
        for _ in range(nb):
            sc = rng.integers(-15, 16, 16).astype(np.int8).tobytes()
            out += bytes(rng.integers(0, 256, 192, dtype=np.uint8)) + sc + (0x1C00).to_bytes(2, "little")
    else:  # Q4_K / Q5_K: d, dmin, 12 scale bytes, (Q5_K: 32 high-bit bytes), 128 nibble bytes
        for _ in range(nb):
            out += (0x1C00).to_bytes(2, "little") + (0x1800).to_bytes(2, "little")
            out += bytes(rng.integers(0, 256, 12 + (32 if fm == em.Q5_K else 0) + 128, dtype=np.uint8))
    return np.frombuffer(bytes(out), np.uint8).copy()


@pytest.mark.parametrize("fm", [em.Q8_0, em.Q4_K, em.Q5_K, em.Q6_K])
def test_q8_block_dots_exact_against_float64(fm):
    """every format's q8 block dot (mx_blk, host/llb_pf.cuh:468-515) equals float64 of the dequantised row
    (the decoders pinned against the reference build above) times x, on inputs where f32 is exact: a
    dropped term, a wrong nibble, scale or sign changes the value"""
    rng = np.random.default_rng(int(fm) + 70)
    cols = 512
    for _ in range(8):
        row = _exact_row(rng, fm, cols)
        _, x = _q4k_exact_case(rng, cols // 256)
        q, d, s = _q8_1(x)
        w = np.zeros(cols, np.float32)
        lib.mo_deq_row(fm, ol.ptr(row), cols, ol.ptr(w))
        exact = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
        assert lib.mo_dot_q8(fm, ol.ptr(row), cols, ol.ptr(q), ol.ptr(d), ol.ptr(s)) == exact
