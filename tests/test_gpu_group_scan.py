"""The dispatch permutation's histogram + scan pair (llb_moe_hip_set_group_scan(1)) on the GPU: off / xmap /
inv equal to the oracle's mo_group (the stable order) and to the per-expert-scan kernel, on uniform, Zipf-
skewed and single-expert slot sets, through llb_moe_hip_group; and a whole f16-tier layer giving the same bits
with either dispatch. Skipped unless LLB_TEST_GROUP_SCAN=1 until the pair has run on a GPU once; its indexing
is restated on the host in test_group_scan_host.py."""
import os

import numpy as np
import pytest

import eureka_moe as em
import oracle_lib as ol
from test_gpu_parity import _say
from test_group_scan_host import CASES, _oracle

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(os.environ.get("LLB_TEST_GROUP_SCAN") != "1",
                                 reason="the histogram + scan dispatch has not run on a GPU yet "
                                        "(LLB_TEST_GROUP_SCAN=1 runs it)")]


def _group(dev, ids, nk, ne, scan):
    dev.check(dev.lib.llb_moe_hip_set_group_scan(1 if scan else 0))
    try:
        n = ids.size
        sb = dev.lib.llb_moe_hip_group_scratch_bytes(n, ne)
        pi = dev.upload(np.ascontiguousarray(ids, np.uint32))
        off, xm, inv, sc = dev.alloc((ne + 1) * 4), dev.alloc(n * 4), dev.alloc(n * 4), dev.alloc(sb)
        dev.check(dev.lib.llb_moe_hip_group(pi, n, nk, ne, off, xm, inv, sc, sb))
        out = dev.read(off, ne + 1, np.uint32), dev.read(xm, n, np.uint32), dev.read(inv, n, np.uint32)
        for p in (pi, off, xm, inv, sc):
            dev.free(p)
        return out
    finally:
        dev.check(dev.lib.llb_moe_hip_set_group_scan(0))


@pytest.mark.parametrize("case", sorted(CASES))
def test_group_scan_matches_the_oracle(dev, case):
    ids, nk, ne = CASES[case]()
    ids = np.asarray(ids, np.uint32)
    _say("group scan", case, ids.size, nk, ne)
    go, gx, gv = _group(dev, ids, nk, ne, True)
    ro, rx, rv = _oracle(ids, nk, ne)
    assert np.array_equal(go, ro) and np.array_equal(gx, rx) and np.array_equal(gv, rv)
    po, px, pv = _group(dev, ids, nk, ne, False)
    assert np.array_equal(go, po) and np.array_equal(gx, px) and np.array_equal(gv, pv)


@pytest.mark.parametrize("name,T", [("c1", 2048), ("c5", 513)])
def test_f16_layer_same_bits_with_either_dispatch(dev, name, T):
    shape = em.SHAPES[name]
    _say("f16 layer, both dispatches", name, T)
    layer = em.Layer(dev, shape, seed=11)
    layer.pack()
    outs = []
    for scan in (0, 1):
        dev.check(dev.lib.llb_moe_hip_set_group_scan(scan))
        try:
            run = em.Runner(dev, shape, T, tier=em.F16)
            run.gen_inputs(11)
            run.forward(layer)
            outs.append(run.outputs())
            run.free()
        finally:
            dev.check(dev.lib.llb_moe_hip_set_group_scan(0))
    layer.free()
    for a, b in zip(*outs):
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))
