"""Writes tests/golden/moe_golden.npz: small seeded MoE layers (weights regenerate from the seed
through the shared generator, so only inputs' seeds, shapes and outputs are stored) with the exact
tier's ids, weights and layer outputs from the CPU oracle. Run from the repo root:
    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.dirname(HERE), os.path.join(os.path.dirname(os.path.dirname(HERE)), "eureka-engine_amd")]
import eureka_moe as em  # noqa: E402
import oracle_lib as ol  # noqa: E402

CASES = [
    # name, shape args, seed, T
    ("q4k_q6k_shared", (2048, 8, 2, 256, 256, em.Q4_K, em.Q4_K, em.Q6_K), 11, 2),
    ("q8_0_noshared", (2048, 8, 2, 256, 0, em.Q8_0, em.Q8_0, em.Q8_0), 12, 2),
    ("q5k_mixed", (2048, 12, 3, 256, 256, em.Q5_K, em.Q5_K, em.Q4_K, em.Q6_K, em.Q6_K, em.Q4_K), 13, 2),
    ("q6k_q8_0", (2048, 6, 4, 512, 0, em.Q6_K, em.Q6_K, em.Q8_0), 14, 1),
]


def main():
    out = {}
    for name, args, seed, T in CASES:
        shape = em.Shape(*args)
        h2, x1 = ol.inputs(shape, seed, T)
        hl = ol.HostLayer(shape, seed=seed, experts=[])
        y, ids, wt, sgo = hl.run(h2, x1)
        out[name + "/shape"] = np.array(list(args), np.uint32)
        out[name + "/seed_T"] = np.array([seed, T], np.uint32)
        out[name + "/ids"] = ids
        out[name + "/wt"] = wt
        out[name + "/sgo"] = sgo
        out[name + "/y"] = y
    np.savez_compressed(os.path.join(HERE, "moe_golden.npz"), **out)
    print("wrote", len(CASES), "cases")


if __name__ == "__main__":
    main()
