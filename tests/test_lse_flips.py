"""LSE parity against the reference's published matmul semantics (fp32 sums of exact bf16
products, order unspecified: attention.metal:93-106, 113), not only against the GPU's own
matrix-core order.

The oracle is run with three accumulation orders for Q.K^T: GEMM_SEQ (plain sequential fp32),
GEMM_CHUNK16 and GEMM_MFMA (gfx950's matrix-core passes, which the GPU kernels execute). Every
row whose LSE moves by more than the 1e-3 bar between two orders must be a diagnosed rounding
flip (tests/lse_flips.py): a score whose exact product lies within fp32 summation error of a bf16
rounding midpoint, whose one-ulp move explains the LSE difference exactly. A planted mistake
(oracle built with scale 1/D) must not pass as a flip.
"""
import numpy as np
import pytest

import oracle as O
from tests.lse_flips import diagnose_row, rows_beyond

MODELS = (O.GEMM_SEQ, O.GEMM_CHUNK16, O.GEMM_MFMA)


def _inputs(B, T, H, D, seed, s):
    return (O.normal_bf16((B, T, H, D), seed, O.TID_Q, s), O.normal_bf16((B, T, H, D), seed, O.TID_K, s),
            O.normal_bf16((B, T, H, D), seed, O.TID_V))


@pytest.mark.parametrize("B,T,H,D,s,seed,max_rows", [
    (2, 1024, 12, 64, 1.5, 22, 3),   # config 2 slice (batches 0-1), the GPU test's inputs
    (1, 4096, 16, 128, 1.0, 23, 0),  # config 3 slice (batch 0, all 16 heads)
])
def test_lse_rows_beyond_bar_are_diagnosed_flips(B, T, H, D, s, seed, max_rows):
    q, k, v = _inputs(B, T, H, D, seed, s)
    lse = {m: O.forward(q, k, v, O.opts(gemm_model=m, threads=8))[1] for m in MODELS}
    seen = 0
    for i, a in enumerate(MODELS):
        for b in MODELS[i + 1:]:
            rows = rows_beyond(lse[a], lse[b])
            for r in rows:
                info = diagnose_row(q, k, lse[a], lse[b], *r, a, b)
                print(f"models {a}/{b}: {info}")
                assert info["flips"], r
                assert abs(info["observed"]) <= info["max_score_step"] * info["flip_weight"] + 5e-5
            seen = max(seen, len(rows))
    assert seen <= max_rows


def test_diagnosis_rejects_a_planted_mistake():
    q, k, v = _inputs(1, 256, 1, 64, 22, 1.5)
    _, good = O.forward(q, k, v, O.opts(gemm_model=O.GEMM_SEQ))
    _, bad = O.Oracle(O.build_mutant(2)).forward(q, k, v, O.opts(gemm_model=O.GEMM_SEQ))
    rows = rows_beyond(good, bad)
    assert rows
    with pytest.raises(AssertionError):
        diagnose_row(q, k, good, bad, *rows[0], O.GEMM_SEQ, O.GEMM_SEQ)
