"""llb_moe_hip_forward_static: the forward with its scratch in the library's static device array (no
allocation, no scratch argument). Through the C ABI on the GPU it must give llb_moe_hip_forward's bits on
two calls in a row, the second on a smaller input (the array keeps the first call's contents), for the
exact and the q8 tiers."""
import ctypes as C

import numpy as np
import pytest

import eureka_moe as em


def _say(*a):
    print(*a, flush=True)


def _both(dev, shape, T, tier, seed):
    layer = em.Layer(dev, shape, seed=seed)
    run = em.Runner(dev, shape, T, tier=tier)
    run.gen_inputs(seed)
    dev.check(dev.lib.llb_moe_hip_forward_static(C.byref(layer.desc), T, run.h2, run.x1, run.y, run.ids, run.wt, tier))
    st = run.outputs()
    run.forward(layer)
    ref = run.outputs()
    run.free()
    layer.free()
    return st, ref


@pytest.mark.gpu
@pytest.mark.parametrize("tier", [em.EXACT, em.Q8])
def test_static_scratch_matches_forward_twice(dev, tier):
    for name, T in (("c5", 3), ("c2", 1)):  # the second call smaller than the first
        _say("forward_static", name, "T", T, "tier", tier)
        (ys, ids_s, wt_s), (yr, ids_r, wt_r) = _both(dev, em.SHAPES[name], T, tier, seed=17 + T)
        assert np.array_equal(ids_s, ids_r)
        assert np.array_equal(wt_s.view(np.uint32), wt_r.view(np.uint32))
        assert np.array_equal(ys.view(np.uint32), yr.view(np.uint32))


@pytest.mark.gpu
def test_static_scratch_refuses_what_it_cannot_hold(dev):
    shape = em.SHAPES["c1"]
    layer = em.Layer(dev, shape, seed=1)
    T = 4096
    probe = em.MoeLayer(shape.dm, shape.ne, shape.nk, shape.ef, shape.sf, shape.fx, shape.fsg, shape.fsu, shape.fsd)
    assert dev.lib.llb_moe_hip_scratch_bytes(C.byref(probe), T, em.EXACT) > em.STATIC_SCRATCH_BYTES
    rc = dev.lib.llb_moe_hip_forward_static(C.byref(layer.desc), T, 0, 0, 0, 0, 0, em.EXACT)
    assert rc == -1 and b"static array" in dev.lib.llb_hip_last_error()
    assert dev.lib.llb_moe_hip_forward_static(C.byref(layer.desc), 1, 0, 0, 0, 0, 0, em.F16) == -1
    layer.free()
