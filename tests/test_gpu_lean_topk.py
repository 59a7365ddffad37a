"""The one-token decode's lean top-k (llb_moe_hip_set_lean_topk(1): four barriers, places and ranks counted
by readlane) on the GPU: ids, weights and layer outputs bit for bit against the oracle on the tie patterns
(the router rows zeroed so the per-expert bias is the logit row) and on configs 1 and 2, and the same bits
as the default top-k. Skipped unless LLB_TEST_LEAN_TOPK=1 until the variant has run on a GPU once; it is
restated on the host in test_topk_lean_host.py."""
import os

import numpy as np
import pytest

import eureka_moe as em
import oracle_lib as ol
from test_gpu_parity import _say, _tie_rows

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(os.environ.get("LLB_TEST_LEAN_TOPK") != "1",
                                 reason="the lean top-k has not run on a GPU yet (LLB_TEST_LEAN_TOPK=1 runs it)")]


@pytest.fixture
def lean(dev):
    dev.check(dev.lib.llb_moe_hip_set_lean_topk(1))
    yield
    dev.check(dev.lib.llb_moe_hip_set_lean_topk(0))


@pytest.mark.parametrize("ne,nk", [(256, 8), (128, 8), (200, 16), (64, 1), (130, 15)])
def test_lean_topk_patterns(dev, lean, ne, nk):
    shape = em.Shape(2048, ne, nk, 256, 256 if nk < 16 else 0, em.Q4_K, em.Q4_K, em.Q6_K)
    rng = np.random.default_rng(ne * 100 + nk)
    rows = _tie_rows(ne, nk, rng)
    layer = em.Layer(dev, shape, seed=11, bias=rows[0])
    dev.check(dev.lib.llb_hip_zero(layer.router, ne * shape.dm * 4))
    run = em.Runner(dev, shape, 1)
    run.gen_inputs(11)
    h2, x1 = ol.inputs(shape, 11, 1)
    hl = ol.HostLayer(shape, seed=11, experts=[], bias=rows[0])
    hl.router[:] = 0
    for k, r in enumerate(rows):
        _say("lean top-k pattern", ne, nk, k)
        dev.write(layer.bias, r)
        run.forward(layer)
        y, ids, wt = run.outputs()
        hl.bias = r.copy()
        hl._mk()
        yr, idr, wtr, _ = hl.run(h2, x1)
        assert np.array_equal(ids, idr), (k, ids, idr)
        assert np.array_equal(wt.view(np.uint32), wtr.view(np.uint32)), k
        assert np.array_equal(y.view(np.uint32), yr.view(np.uint32)), k
    run.free()
    layer.free()


@pytest.mark.parametrize("name", ["c1", "c2"])
def test_lean_topk_configs_same_bits(dev, name):
    shape = em.SHAPES[name]
    _say("lean top-k", name)
    layer = em.Layer(dev, shape, seed=0)
    outs = []
    for on in (0, 1):
        dev.check(dev.lib.llb_moe_hip_set_lean_topk(on))
        try:
            run = em.Runner(dev, shape, 1)
            run.gen_inputs(0)
            run.forward(layer, residual=False)
            outs.append(run.outputs())
            run.free()
        finally:
            dev.check(dev.lib.llb_moe_hip_set_lean_topk(0))
    layer.free()
    for a, b in zip(*outs):
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))
    h2, _ = ol.inputs(shape, 0, 1)
    yr, idr, wtr, _ = ol.HostLayer(shape, seed=0, experts=[]).run(h2, None)
    y, ids, wt = outs[1]
    assert np.array_equal(ids, idr) and np.array_equal(y.view(np.uint32), yr.view(np.uint32))
