"""Diagnosis of logsumexp rows that move under a different fp32 accumulation order of Q.K^T.

The reference rounds every score twice (S = bf16(Q.K^T), attention.metal:113; s = bf16(S*scale),
:115-121), and Apple does not publish the order in which its matmul2d sums the D products in
fp32 (:93-106). A product whose exact value lies within fp32 summation error of a bf16 rounding
midpoint rounds to one neighbour under one summation order and to the other under another: the
score moves by one bf16 ulp (times the scale), and a row whose softmax that score dominates moves
its LSE by up to that amount. Such a flip is a property of the inputs, not a fault of either
order; a 1e-3 LSE bar cannot hold for it across orders.

diagnose_row() proves, for one (b, h, t) row, that the LSE difference between two oracle runs
is exactly that: every score on which the two products disagree is a neighbour pair around a
midpoint within the fp32 error bound of its exact (float64) dot product, and the LSE difference
is what those score changes alone produce (float64 logsumexp of the two rounded score vectors).
"""
from __future__ import annotations

import numpy as np

import oracle as O

f32 = O.bf16_to_f32


def _bf(x):
    return f32(O.f32_to_bf16(np.asarray(x, dtype=np.float32)))


def _scaled(S, D):
    """s = bf16(S * scale): the reference's second rounding (exact for D = 64, scale 1/8)."""
    scale = np.float32(1.0) / np.sqrt(np.float32(D))
    return _bf(S.astype(np.float32) * scale)


def row_scores(q, k, b, h, t, model, layout=O.PASS_SEQ8):
    """bf16(Q.K^T) of query t against keys 0..t under one GEMM model, through the oracle's own dot."""
    orc = O.default()
    qa = f32(q[b, t, h])
    return np.array([_bf(orc.dot(0.0, qa, f32(k[b, j, h]), model, layout)) for j in range(t + 1)], np.float32)


def diagnose_row(q, k, lse_a, lse_b, b, h, t, model_a, model_b, tol=5e-5):
    """Returns a dict describing row (b, h, t); raises AssertionError if the difference of the two
    LSE values is not explained by score flips at bf16 rounding midpoints (to within tol)."""
    D = q.shape[-1]
    Sa = row_scores(q, k, b, h, t, model_a)
    Sb = row_scores(q, k, b, h, t, model_b)
    qa = f32(q[b, t, h]).astype(np.float64)
    K = f32(k[b, :t + 1, h]).astype(np.float64)
    exact = K @ qa
    mag = np.abs(K * qa).sum(1)
    flips = np.nonzero(Sa != Sb)[0]
    for j in flips:
        ba, bb = (int(x) for x in O.f32_to_bf16(np.array([Sa[j].item(), Sb[j].item()], np.float32)))
        # neighbours: same sign, bit patterns one apart (no bf16 value between them)
        assert (ba ^ bb) & 0x8000 == 0 and abs(ba - bb) == 1, (j, hex(ba), hex(bb))
        mid = 0.5 * (float(Sa[j].item()) + float(Sb[j].item()))
        # both models are fp32 sums of D exact products: each is within D*2^-24*sum|terms| of exact
        bound = D * 2.0 ** -24 * mag[j]
        assert abs(exact[j] - mid) <= bound, (j, exact[j], mid, bound)
    sa, sb = _scaled(Sa, D).astype(np.float64), _scaled(Sb, D).astype(np.float64)

    def lse64(s):
        m = s.max()
        return m + np.log(np.exp(s - m).sum())

    explained = lse64(sa) - lse64(sb)
    observed = float(lse_a[b, h, t]) - float(lse_b[b, h, t])
    # softmax weights of the flipped scores, the larger of the two models' (the LSE is monotone in
    # each score with slope equal to its weight, so |observed| <= step * max weight)
    w = np.maximum(np.exp(sa - lse64(sa)), np.exp(sb - lse64(sb)))
    assert abs(observed - explained) <= tol, (b, h, t, observed, explained)
    return {
        "row": (b, h, t), "flips": [int(j) for j in flips], "observed": observed, "explained": float(explained),
        "max_score_step": float(np.abs(sa - sb).max()) if len(flips) else 0.0,
        "flip_weight": float(w[flips].sum()) if len(flips) else 0.0,
        "weights": [float(np.ravel(w)[j]) for j in flips],
        "steps": [float(abs(np.ravel(sa)[j] - np.ravel(sb)[j])) for j in flips],
    }


def o_move_bound(info, v_keys, o_row):
    """Per-column bound on how far the flipped scores of one diagnosed row move its output
    O = sum_i w_i V_i. Moving score j by delta multiplies its unnormalised weight by e^delta, which
    changes O by w_j (e^delta - 1) (V_j - O) / (1 + w_j (e^delta - 1)); summed over the flips with
    |e^delta - 1| <= e^|delta| - 1 and the denominator at its smallest. v_keys: the flipped keys' V
    rows [n_flips, D]; o_row: the reference's unrounded O row [D]. w_j is the larger of the two
    models' weights, so the bound holds from either side."""
    w = np.asarray(info["weights"], np.float64)
    st = np.asarray(info["steps"], np.float64)
    den = 1.0 - float(np.sum(w * -np.expm1(-st)))
    num = np.sum((w * np.expm1(st))[:, None] * np.abs(np.asarray(v_keys, np.float64) - np.asarray(o_row, np.float64)[None, :]),
                 axis=0)
    return num / den


def rows_beyond(lse_a, lse_b, bar=1e-3):
    idx = np.argwhere(np.abs(lse_a - lse_b) > bar)
    return [tuple(int(x) for x in r) for r in idx]
