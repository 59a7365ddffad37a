"""llb_rmsnorm_add, the step before the router (tools/payload-fuse.patch:106-127): the oracle's restatement
pinned by (1) an independent pairwise tree written here in numpy, over the next power of two >= n with +0
leaves, (2) the reference CPU twin's rms_norm (tools/qwen35_engine.c:510-515, compiled from the reference
checkout into oracle/_ref) on inputs whose squares and sums are exact in any order, so every order gives
the same bits -- this pins the formula and the order of the final ops -- and (3) float64. The GPU kernel is
checked bit for bit against the oracle in test_gpu_parity.py."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as ol

EPS = np.float32(1e-6)


def tree_np(v):
    """balanced pairwise sum in index order over the next power of two >= len(v), +0 leaves"""
    P = 1
    while P < len(v):
        P *= 2
    a = np.zeros(P, np.float32)
    a[:len(v)] = v
    while len(a) > 1:
        a = (a[0::2] + a[1::2]).astype(np.float32)
    return a[0]


@pytest.mark.parametrize("n", [1, 3, 256, 1024, 1536, 2048, 4096, 5120])
def test_oracle_tree_order(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((2, n)) * 3).astype(np.float32)
    z = rng.standard_normal((2, n)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    x1, h2, s = ol.rmsnorm_add(x, z, w, EPS)
    for t in range(2):
        v = (x[t] + z[t]).astype(np.float32)
        assert np.array_equal(x1[t].view(np.uint32), v.view(np.uint32))
        ss = tree_np((v * v).astype(np.float32))
        st = np.float32(1.0) / np.sqrt(np.float32(ss / np.float32(n)) + EPS, dtype=np.float32)
        assert s[t].view(np.uint32) == np.float32(st).view(np.uint32)
        want = ((v * st).astype(np.float32) * w).astype(np.float32)
        assert np.array_equal(h2[t].view(np.uint32), want.view(np.uint32))


def test_tree_order_is_not_sequential():
    """an input on which the sequential and the tree sums differ, so the order above is a real check"""
    n = 2048
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((1, n)) * 10 ** rng.uniform(-3, 3, n)).astype(np.float32)
    z = np.zeros_like(x)
    seq = np.float32(0)
    for v in x[0]:
        seq = np.float32(seq + np.float32(v * v))
    assert seq != tree_np((x[0] * x[0]).astype(np.float32))


def test_against_reference_cpu_twin_on_exact_sums():
    ref = ol.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    rng = np.random.default_rng(3)
    for n in (1024, 2048, 4096):
        x = rng.integers(-40, 41, (1, n)).astype(np.float32)   # squares <= 1600, sums < 2^24: exact
        z = rng.integers(-8, 9, (1, n)).astype(np.float32)
        w = rng.standard_normal(n).astype(np.float32)
        _, h2, _ = ol.rmsnorm_add(x, z, w, EPS)
        v = (x[0] + z[0]).astype(np.float32)
        hr = np.zeros(n, np.float32)
        ref.ref_rms_norm(ol.ptr(hr), ol.ptr(v), ol.ptr(w), n, C.c_float(EPS))
        assert np.array_equal(h2[0].view(np.uint32), hr.view(np.uint32))


def test_float64_and_special_rows():
    rng = np.random.default_rng(5)
    n = 2048
    x = rng.standard_normal((3, n)).astype(np.float32)
    z = rng.standard_normal((3, n)).astype(np.float32)
    x[2] = 0.0
    z[2] = 0.0                                   # a zero row: s = 1 / sqrt(eps), h2 = +0
    w = rng.standard_normal(n).astype(np.float32)
    x1, h2, s = ol.rmsnorm_add(x, z, w, EPS)
    v = x.astype(np.float64) + z.astype(np.float64)
    s64 = 1.0 / np.sqrt((v[:2] ** 2).mean(axis=1) + float(EPS))
    ref = v[:2] * s64[:, None] * w
    assert np.abs(h2[:2] - ref).max() / np.abs(ref).max() < 1e-5
    assert s[2] == np.float32(1.0) / np.sqrt(EPS, dtype=np.float32)
    assert not np.signbit(h2[2][w > 0]).any() and (h2[2] == 0).all()


def test_c_abi_rejects_bad_widths_without_a_device():
    """the entry point's argument rules are checked on the host, before any device call"""
    import eureka_moe as em
    lib = em.load()
    fake = 1 << 40   # never dereferenced: every call below fails its checks first
    for T, n in ((1, 0), (1, 16385), (0, 2048), (1, 1030)):
        assert lib.llb_moe_hip_rmsnorm_add(fake, fake, fake, 1e-6, T, n, 0, fake) != 0
    assert b"rmsnorm_add" in lib.llb_hip_last_error()
    assert lib.llb_moe_hip_rmsnorm_add(0, fake, fake, 1e-6, 1, 2048, 0, fake) != 0
