"""GPU parity: the HIP kernels through the C ABI against the CPU oracle on identical seeded inputs.

Bars: LSE within 1e-3; O within 1e-2 max-abs, except elements whose
bf16 spacing exceeds 1e-2 (|O| >= 2), where the bar is one bf16 ulp; dQ/dK/dV within 2e-2
max-abs relative to max |grad|; computeD bit-exact (same inputs, same summation order).
"""
import numpy as np
import pytest

import oracle as O
from tests.attn_case import (gpu_backward, gpu_compute_d, gpu_forward, make_inputs, oracle_all, out_error,
                             rel_to_max, f32)

pytestmark = pytest.mark.gpu

CASES = [
    # (B, T, H, D, qk_scale, seed)
    (16, 256, 6, 64, 1.0, 11),    # config 0 shape (the reference default)
    (2, 512, 2, 128, 1.0, 12),    # D=128
    (1, 1024, 12, 64, 1.5, 13),   # config 2 slice: peaky rows
    (1, 192, 3, 128, 1.5, 14),    # T not a multiple of 128, peaky
]


@pytest.mark.parametrize("B,T,H,D,s,seed", CASES)
def test_forward_backward_parity(gpu, B, T, H, D, s, seed):
    print(f"case B={B} T={T} H={H} D={D} qk_scale={s} seed={seed}", flush=True)
    q, k, v, g = make_inputs(B, T, H, D, seed, s)
    ref = oracle_all(q, k, v, g)
    out, lse = gpu_forward(q, k, v, gpu)
    lse_err = float(np.abs(lse - ref["lse"]).max())
    o_max, o_bad, o_over = out_error(out, ref["out"])
    print(f"  fwd: lse max err {lse_err:.3g}, O max err {o_max:.3g}, O beyond bar {o_bad}, O > 1e-2 {o_over}")
    assert lse_err <= 1e-3
    assert o_bad == 0
    # computeD on the oracle's O: same inputs, same order -> bit-exact
    Dg = gpu_compute_d(g, ref["out"], gpu)
    assert np.array_equal(Dg, ref["D"]), f"computeD differs: {np.abs(Dg - ref['D']).max()}"
    # backward on the oracle's lse and D
    dQ, dK, dV = gpu_backward(g, ref["D"], ref["lse"], q, k, v, gpu)
    errs = {n: rel_to_max(x, ref[n]) for n, x in (("dQ", dQ), ("dK", dK), ("dV", dV))}
    print("  bwd rel-to-max:", {n: f"{e:.3g}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= 2e-2, n
