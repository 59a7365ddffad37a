"""Known-answer pins for the four layer steps the oracle restates from the reference's kernel text:
the combine (tools/payload-moeany.patch:572-592), SwiGLU (:495), the renormalisation (:459-467) and the
shared gate's sigmoid (:468).

Every case is built from powers of two (or values whose products are followed by hand), so the expected
bits are derived in the docstrings, not recomputed by the oracle's formula; each case also carries the
plausible mistakes (another summation order, a fused multiply-add, a reciprocal, a 0 + v0 wt0 start, no
clamp, the residual added before the shared expert) and asserts that every one of them gives other bits,
so a reassociation in the oracle fails here. SwiGLU and the sigmoid are also pinned bit for bit against the
reference's own compiled hf_silu / hf_sigmoid (tools/qwen35_engine.c:49-50, built into oracle/_ref), whose
dense FFN applies silu(g) * u exactly as the MoE kernel does (tools/qwen35_engine.c:744).
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle_lib as ol

lib = ol.lib()
F = np.float32


def b(x):
    return int(np.asarray(x, np.float32).view(np.uint32))


def combine(v, wt, shared=False, hv=0.0, sgo=0.0, res=0.0):
    v, wt = np.ascontiguousarray(v, F), np.ascontiguousarray(wt, F)
    return F(lib.mo_combine(ol.ptr(v), ol.ptr(wt), v.size, int(shared), float(hv), float(sgo), float(res)))


def renorm(wt):
    w = np.ascontiguousarray(wt, F).copy()
    lib.mo_renorm(ol.ptr(w), w.size)
    return w


# ---- mutants: the orders a restatement could plausibly take instead (float32 at every step)

def seq(terms):
    s = terms[0]
    for t in terms[1:]:
        s = F(s + t)
    return s


def m_zero_start(v, wt):
    s = F(0.0)
    for a, c in zip(v, wt):
        s = F(s + F(F(a) * F(c)))
    return s


def m_reverse(v, wt):
    p = [F(F(a) * F(c)) for a, c in zip(v, wt)]
    return seq(p[::-1])


def m_pairwise(v, wt):
    p = [F(F(a) * F(c)) for a, c in zip(v, wt)]
    while len(p) > 1:
        p = [F(p[i] + p[i + 1]) if i + 1 < len(p) else p[i] for i in range(0, len(p), 2)]
    return p[0]


def m_fma(v, wt):
    """mo + v wt rounded once (a contracted multiply-add), from the first product on"""
    s = F(F(v[0]) * F(wt[0]))
    for a, c in zip(v[1:], wt[1:]):
        s = F(Fraction(float(s)) + Fraction(float(a)) * Fraction(float(c)))
    return s


# ---------------------------------------------------------------- combine

def test_combine_rank_order_sequential():
    """v = 1 x4, wt = (2^24, 1, 1, 1), no shared expert, residual 0.
    Rank order: 2^24 + 1 is a tie between 2^24 and 2^24 + 2 (spacing 2 above 2^24), to even: 2^24; twice
    more the same: y = 2^24.
    Pairwise: (2^24 + 1) + (1 + 1) = 2^24 + 2. Reverse: 1 + 1 + 1 = 3, 3 + 2^24 ties to 2^24 + 4."""
    v, wt = [1, 1, 1, 1], [2.0 ** 24, 1, 1, 1]
    want = F(2.0 ** 24)
    assert b(combine(v, wt)) == b(want)
    assert m_pairwise(v, wt) == F(2.0 ** 24 + 2)
    assert m_reverse(v, wt) == F(2.0 ** 24 + 4)


def test_combine_shared_before_residual():
    """nk = 1: v0 wt0 = 2^24; the shared term hv sgo = 1, the residual 2.
    (2^24 + 1) ties to 2^24, + 2 = 2^24 + 2 (exact).
    Residual first: 2^24 + 2, + 1 = 2^24 + 3, a tie, to even 2^24 + 4. Shared + residual first: 3, + 2^24 =
    2^24 + 4 (tie to even)."""
    got = combine([1], [2.0 ** 24], shared=True, hv=1, sgo=1, res=2)
    want = F(2.0 ** 24 + 2)
    assert b(got) == b(want)
    assert F(F(F(2.0 ** 24) + F(2)) + F(1)) != want
    assert F(F(2.0 ** 24) + F(F(1) + F(2))) != want


def test_combine_products_round_before_the_add():
    """v = (-1, 1 + 2^-23), wt = (1, 1 + 2^-23): the second product is 1 + 2^-22 + 2^-46, which rounds to
    1 + 2^-22; -1 + that = 2^-22 exactly. A fused multiply-add keeps 2^-22 + 2^-46 (representable).
    The same through the shared term: mo = -1, hv = sgo = 1 + 2^-23 gives 2^-22."""
    e = 1 + 2.0 ** -23
    v, wt = [-1, e], [1, e]
    assert b(combine(v, wt)) == b(F(2.0 ** -22))
    assert m_fma(v, wt) == F(2.0 ** -22 + 2.0 ** -46)
    got = combine([-1], [1], shared=True, hv=e, sgo=e, res=0)
    assert b(got) == b(F(2.0 ** -22))


def test_combine_starts_from_the_first_product():
    """All products -0 and the residual -0: mo = v0 wt0 = -0, -0 + -0 = -0, y = -0 (sign bit set).
    Starting from 0.0f instead gives +0 (+0 + -0 = +0 in round-to-nearest)."""
    v, wt = [-0.0, -0.0], [1, 1]
    assert b(combine(v, wt, res=-0.0)) == 0x80000000
    assert b(F(m_zero_start(v, wt) + F(-0.0))) == 0


def test_combine_k_terms_in_rank_order_against_exact_rationals():
    """A denser check of the same order: random products whose f32 sum in rank order is followed with exact
    rationals (each product and each partial sum rounded to nearest even once, via float64, which is exact
    for one f32 operation); pairwise and reverse orders disagree on a good share of them."""
    rng = np.random.default_rng(5)
    diff_pair = diff_rev = 0
    for _ in range(300):
        nk = int(rng.integers(2, 11))
        v = (rng.standard_normal(nk) * 2.0 ** rng.integers(-4, 8, nk)).astype(F)
        wt = rng.random(nk).astype(F)
        res, hv, so = F(rng.standard_normal()), F(rng.standard_normal()), F(rng.random())
        mo = F(float(v[0]) * float(wt[0]))
        for j in range(1, nk):
            mo = F(float(mo) + float(F(float(v[j]) * float(wt[j]))))
        want = F(float(F(float(mo) + float(F(float(hv) * float(so))))) + float(res))
        got = combine(v, wt, shared=True, hv=hv, sgo=so, res=res)
        assert b(got) == b(want)
        diff_pair += m_pairwise(v, wt) != mo
        diff_rev += m_reverse(v, wt) != mo
    assert diff_pair > 20 and diff_rev > 20, (diff_pair, diff_rev)


# ---------------------------------------------------------------- renormalisation

def test_renorm_rank_order_sum():
    """wt = (1, 2^-24, 2^-24): 1 + 2^-24 ties to 1 (spacing 2^-23 above 1), twice: s = 1, wt unchanged.
    Summed from the smallest: 2^-24 + 2^-24 = 2^-23, + 1 = 1 + 2^-23 exactly, and wt0 / s = 1 - 2^-23."""
    got = renorm([1, 2.0 ** -24, 2.0 ** -24])
    assert [b(x) for x in got] == [b(F(1)), b(F(2.0 ** -24)), b(F(2.0 ** -24))]
    s_rev = F(F(F(2.0 ** -24) + F(2.0 ** -24)) + F(1))
    assert s_rev == F(1 + 2.0 ** -23) and F(F(1) / s_rev) == F(1 - 2.0 ** -23)


def test_renorm_clamp_at_2_pow_minus_14():
    """wt = (2^-16, 2^-17): s = 3 * 2^-17 < 2^-14, so s = 2^-14 and wt = (1/4, 1/8); without the clamp
    (2/3, 1/3). At the threshold, wt = (2^-15, 2^-15): s = 2^-14, not below it: (1/2, 1/2)."""
    got = renorm([2.0 ** -16, 2.0 ** -17])
    assert [b(x) for x in got] == [b(F(0.25)), b(F(0.125))]
    got = renorm([2.0 ** -15, 2.0 ** -15])
    assert [b(x) for x in got] == [b(F(0.5)), b(F(0.5))]


def test_renorm_divides():
    """wt = (5, 1): s = 6; 5 / 6 correctly rounded is the f32 nearest 0.8333..., which the exact rational
    gives; 5 * (1 / 6) rounds twice and lands one ulp away."""
    got = renorm([5, 1])

    def rn(q):
        return F(float(q))  # q is n / 6 with small n: float64 then f32 is correctly rounded here

    assert b(got[0]) == b(rn(Fraction(5, 6))) and b(got[1]) == b(rn(Fraction(1, 6)))
    assert F(F(5) * F(F(1) / F(6))) != got[0]


def test_topk_uses_the_renorm_and_sigmoid():
    """mo_topk's weights are the renormalised top-k probabilities and its sgo the sigmoid. Logits (0, x, x)
    with v1 = exp(x) (through double) in (2^-25, 2^-24): after the max shift v = (1, v1, v1); the softmax
    total is 1 (1 + v1 is below the tie at 1 + 2^-24, twice), so p = v, and the rank-order renorm sum is 1
    again: wt = (1, v1, v1). Summed from the smallest, 2 v1 + 1 is above the tie and gives 1 + 2^-23, so
    wt0 would be 1 - 2^-23."""
    x = F(-24 * np.log(2) - 0.1)
    v1 = F(np.exp(np.float64(x)))
    assert F(2.0 ** -25) < v1 < F(2.0 ** -24)
    lg = np.array([0.0, x, x], F)
    ids, wt, sgo = np.zeros(3, np.uint32), np.zeros(3, F), np.zeros(1, F)
    lib.mo_topk(ol.ptr(lg), 3, 3, 0.75, ol.ptr(ids), ol.ptr(wt), ol.ptr(sgo))
    assert list(ids) == [0, 1, 2]
    assert [b(w) for w in wt] == [b(F(1)), b(v1), b(v1)]
    assert F(F(F(v1 + v1) + F(1))) == F(1 + 2.0 ** -23)
    assert b(sgo[0]) == b(F(lib.mo_sigmoid(0.75)))


# ---------------------------------------------------------------- SwiGLU and the sigmoid

def _ref():
    r = ol.ref_lib()
    if r is None:
        pytest.skip("oracle/_ref/libref_q35.so is not built (make -C oracle ref; needs the reference tree)")
    return r


def _samples(n, seed):
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(n) * 2.0 ** rng.integers(-6, 5, n)).astype(F)
    g[:8] = [0.0, -0.0, 1.0, -1.0, 20.0, -20.0, 88.0, -88.0]
    u = (rng.standard_normal(n) * 2.0 ** rng.integers(-6, 5, n)).astype(F)
    return g, u


def test_silu_mul_is_the_reference_silu_times_u():
    """silu(g) * u: the reference's hf_silu(g) = g / (1 + exp(-g)) (exp through double), then one f32
    multiply by u (tools/qwen35_engine.c:744, tools/payload-moeany.patch:495). Mutants: g * sigmoid(g) * u,
    g * (u / (1 + e)), (g * u) / (1 + e) each give other bits on part of the sample."""
    r = _ref()
    g, u = _samples(20000, 1)
    got = np.array([lib.mo_silu_mul(float(a), float(c)) for a, c in zip(g, u)], F)
    want = np.array([F(F(r.ref_hf_silu(float(a))) * c) for a, c in zip(g, u)], F)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    e = np.array([F(np.exp(-np.float64(a))) for a in g], F)
    one = F(1)
    mutants = {
        "g*sig*u": F(g * F(one / F(one + e))) * u,
        "g*(u/(1+e))": g * F(u / F(one + e)),
        "(g*u)/(1+e)": F(g * u) / F(one + e),
    }
    with np.errstate(all="ignore"):
        for name, m in mutants.items():
            m = np.asarray(m, F)
            assert np.count_nonzero(m.view(np.uint32) != want.view(np.uint32)) > 100, name


def test_sigmoid_is_the_reference_hf_sigmoid():
    """sgo = 1 / (1 + exp(-sg)), exp through double: bit for bit the reference's hf_sigmoid; the mutants
    exp(x) / (1 + exp(x)) and a float32 exp give other bits on part of the sample."""
    r = _ref()
    g, _ = _samples(20000, 2)
    got = np.array([lib.mo_sigmoid(float(a)) for a in g], F)
    want = np.array([r.ref_hf_sigmoid(float(a)) for a in g], F)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with np.errstate(all="ignore"):
        ep = np.array([F(np.exp(np.float64(a))) for a in g], F)
        m1 = ep / F(F(1) + ep)
        m2 = F(1) / F(F(1) + np.exp(-g))  # float32 exp
    assert np.count_nonzero(np.asarray(m1, F).view(np.uint32) != want.view(np.uint32)) > 100
    assert np.count_nonzero(np.asarray(m2, F).view(np.uint32) != want.view(np.uint32)) > 10
