"""The committed golden vectors (tests/golden/moe_golden.npz, written by make_golden.py): the oracle
must keep reproducing them (CPU), and the HIP exact tier must reproduce them bit for bit (GPU)."""
import os

import numpy as np
import pytest

import eureka_moe as em
import oracle_lib as ol

G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "moe_golden.npz"))
NAMES = sorted({k.split("/")[0] for k in G.files})


def _case(name):
    shape = em.Shape(*[int(v) for v in G[name + "/shape"]])
    seed, T = (int(v) for v in G[name + "/seed_T"])
    return shape, seed, T


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_golden(name):
    shape, seed, T = _case(name)
    h2, x1 = ol.inputs(shape, seed, T)
    y, ids, wt, sgo = ol.HostLayer(shape, seed=seed, experts=[]).run(h2, x1)
    assert np.array_equal(ids, G[name + "/ids"])
    assert np.array_equal(wt.view(np.uint32), G[name + "/wt"].view(np.uint32))
    assert np.array_equal(y.view(np.uint32), G[name + "/y"].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_hip_reproduces_golden(dev, name):
    shape, seed, T = _case(name)
    print("golden", name, flush=True)
    layer = em.Layer(dev, shape, seed=seed)
    run = em.Runner(dev, shape, T)
    run.gen_inputs(seed)
    run.forward(layer)
    y, ids, wt = run.outputs()
    run.free()
    layer.free()
    assert np.array_equal(ids, G[name + "/ids"])
    assert np.array_equal(wt.view(np.uint32), G[name + "/wt"].view(np.uint32))
    assert np.array_equal(y.view(np.uint32), G[name + "/y"].view(np.uint32))
