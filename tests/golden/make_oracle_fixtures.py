"""Writes the oracle regression fixtures tests/golden/oracle_<case>.npz: the seeded inputs (Q, K,
V, dO as bf16 bits) and the CPU oracle's outputs on them (O, LSE, D, dQ, dK, dV; default matrix
product model, the reference's rounding points) at B=1, H=2, T=128, D in {64, 128}, with Q and K
at scale 1 and at x1.5 (peaky rows).

They are data, not a reference run: they pin the oracle and the input generator against their
own earlier outputs, so that a refactor of either shows up as a fixture mismatch
(tests/test_oracle.py), and they give the GPU parity tests committed inputs and expected outputs
(tests/test_gpu_parity.py).

    python tests/golden/make_oracle_fixtures.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.attn_case import make_inputs, oracle_all  # noqa: E402

# (name, D, qk_scale, seed)
CASES = [("d64", 64, 1.0, 501), ("d64_peaky", 64, 1.5, 502), ("d128", 128, 1.0, 503), ("d128_peaky", 128, 1.5, 504)]
B, T, H = 1, 128, 2


def path_of(name):
    return os.path.join(HERE, f"oracle_{name}.npz")


def main():
    for name, D, s, seed in CASES:
        q, k, v, g = make_inputs(B, T, H, D, seed, s)
        r = oracle_all(q, k, v, g)
        np.savez_compressed(path_of(name), seed=np.int64(seed), qk_scale=np.float64(s), q=q, k=k, v=v, dO=g, **r)
        print("wrote", path_of(name), os.path.getsize(path_of(name)), "bytes")


if __name__ == "__main__":
    main()
