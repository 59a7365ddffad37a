"""The f16 tier's in-wave pipelined GEMM body (LLB_MOE_GEMM_PIPE=1, packed stacks) against the default
body: the same products in the same order, so the same bits, for every weight format, the shared
expert, ragged expert tiles and k-tile counts that are not a multiple of the six-step round."""
import os

import numpy as np
import pytest

import eureka_moe as em

pytestmark = pytest.mark.gpu

# every expert format (Q8_0, Q4_K, Q5_K, Q6_K), K = 256 / 512 / 768 / 1280+256 / 2048 / 4096
SMALL = [
    em.Shape(2048, 32, 4, 256, 256, em.Q4_K, em.Q4_K, em.Q6_K),
    em.Shape(2048, 64, 6, 256, 512, em.Q5_K, em.Q5_K, em.Q5_K, fsg=em.Q5_K, fsu=em.Q5_K, fsd=em.Q4_K),
    em.Shape(4096, 40, 8, 512, 256, em.Q6_K, em.Q6_K, em.Q8_0, fsg=em.Q6_K, fsu=em.Q6_K, fsd=em.Q6_K),
    em.Shape(1280 + 256, 1000, 5, 256, 0, em.Q4_K, em.Q4_K, em.Q4_K),
]
CASES = [(s, 150) for s in SMALL] + [("c1", 300), ("c1k", 300), ("c2", 40), ("c1", 2048), ("c5", 1025)]


def _run(dev, shape, T, pipe):
    os.environ["LLB_MOE_GEMM_PIPE"] = "1" if pipe else "0"
    try:
        layer = em.Layer(dev, shape, seed=9)
        layer.pack()
        run = em.Runner(dev, shape, T, tier=em.F16)
        run.gen_inputs(9)
        run.forward(layer)
        out = run.outputs()
        run.free()
        layer.free()
    finally:
        os.environ.pop("LLB_MOE_GEMM_PIPE", None)
    return out


@pytest.mark.parametrize("name,T", CASES)
def test_gemm_pipe_same_bits(dev, name, T):
    shape = em.SHAPES[name] if isinstance(name, str) else name
    print("gemm pipe vs default", name if isinstance(name, str) else vars(name), "T", T, flush=True)
    y0, ids0, wt0 = _run(dev, shape, T, False)
    y1, ids1, wt1 = _run(dev, shape, T, True)
    assert np.array_equal(ids0, ids1) and np.array_equal(wt0.view(np.uint32), wt1.view(np.uint32))
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32)), np.abs(y0 - y1).max()
