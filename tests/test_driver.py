"""The standalone C host (eureka-engine_amd/driver/moe_layer_drv.c): one layer built from its 32 table
words and run through llb_moe_run_table over the C ABI alone, as llb_moe_run would
(host/llb_host.c:622-724). On the GPU its y, ids and wt must be the bits the Python harness gets for the
same seeds through llb_moe_hip_forward -- the table row decodes to the same layer, and nothing outside
the C ABI is needed to drive it. Without a GPU: the binary exists, is linked against the in-tree
library, and refuses bad arguments."""
import os
import subprocess

import numpy as np
import pytest

import eureka_moe as em

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "eureka-engine_amd", "moe_layer_drv")


def _exe():
    if not os.path.exists(EXE):
        pytest.fail("moe_layer_drv is not built (eureka-engine_amd/build.sh builds it)")
    return EXE


def test_driver_refuses_bad_arguments():
    for args in ([], ["c9", "0", "1", "0", "/dev/null"], ["c2", "0", "0", "0", "/dev/null"],
                 ["c2", "0", "1", "7", "/dev/null"]):
        r = subprocess.run([_exe()] + args, capture_output=True, timeout=60)
        assert r.returncode == 2, (args, r.returncode, r.stderr)


def test_driver_links_the_in_tree_library():
    r = subprocess.run(["ldd", _exe()], capture_output=True, text=True, timeout=60)
    lib = [l for l in r.stdout.splitlines() if "libeureka_moe.so" in l]
    assert lib and os.path.join(ROOT, "eureka-engine_amd") in os.path.realpath(lib[0].split("=>")[1].split()[0])


@pytest.mark.gpu
@pytest.mark.parametrize("name,T,tier", [("c2", 1, em.EXACT), ("c2", 5, em.EXACT), ("c2", 2, em.Q8),
                                         ("c2", 64, em.F16), ("c5", 3, em.EXACT)])
def test_driver_matches_the_forward(dev, tmp_path, name, T, tier):
    seed = 11
    out = tmp_path / "y.bin"
    print("driver", name, "T", T, "tier", tier, flush=True)
    r = subprocess.run([_exe(), name, str(seed), str(T), str(tier), str(out)], capture_output=True, text=True,
                       timeout=110)
    assert r.returncode == 0, r.stderr
    shape = em.SHAPES[name]
    raw = np.fromfile(out, np.uint32)
    n, m = T * shape.dm, T * shape.nk
    assert raw.size == n + 2 * m
    yd, idd, wtd = raw[:n].reshape(T, shape.dm), raw[n:n + m].reshape(T, shape.nk), raw[n + m:].reshape(T, shape.nk)
    layer = em.Layer(dev, shape, seed=seed)
    run = em.Runner(dev, shape, T, tier=tier)
    run.gen_inputs(seed)
    run.forward(layer)
    y, ids, wt = run.outputs()
    run.free()
    layer.free()
    assert np.array_equal(idd, ids)
    assert np.array_equal(wtd, wt.view(np.uint32))
    assert np.array_equal(yd, y.view(np.uint32))
