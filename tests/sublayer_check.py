"""Checks every stage of an attention sublayer run on the GPU (per-call chain, phase encoder or graph
replay) against the CPU oracle, on the GPU's own inputs to each stage.

Row-local stages (computeQKV, the attention core, projForward, projBackwarddX, computeD,
computeGradDx) are checked on the rows of the given batches. The weight gradients reduce over all
B*T rows (projBackwarddW, computeGradDw), so they are checked in full against float64 products of
the GPU's own operands, which the oracle's fp32 sums can only approach: bf16 results within one
bf16 ulp of the exact value plus 1e-5 of max|exact| (the fp32 summation error of a 16384-term
sum), fp32 results within 1e-4 of max|exact|.

Reference chain: /root/reference/model.h:446-482 (forward) and :621-690 (backward).
"""
from __future__ import annotations

import numpy as np

import oracle as O
from tests.attn_case import bf16_ulp, f32, rel_to_max, to_np


def bf_err(gpu, ref):
    a, b = f32(gpu), f32(ref)
    d = np.abs(a - b)
    bar = bf16_ulp(b) + 1e-5 * np.abs(b).max()
    return int((d > bar).sum()), float(d.max())


def f32_err(gpu, ref):
    return float(np.abs(gpu - ref).max() / max(np.abs(ref).max(), 1e-30))


def exact_bf_err(gpu_bits, exact):
    """bf16 result against an exact (float64) value: count beyond one ulp + 1e-5 of max."""
    a = f32(gpu_bits).astype(np.float64)
    bar = bf16_ulp(exact.astype(np.float32)).astype(np.float64) + 1e-5 * np.abs(exact).max()
    return int((np.abs(a - exact) > bar).sum())


WEIGHT_GRADS = ("dWq", "dWk", "dWv", "dWp")


def same_up_to_order(name, a, b):
    """Weight gradient `name` of the phase encoder (a) against the per-call chain's (b). The encoder
    computes dWq, dWk, dWv and dProjw in one launch (computeGradDw's kernel with dProjw as a fourth
    weight), over other row chunks than the entry points, so the fp32 sums run in another order:
    dWq (fp32) within 1e-4 of max|b|, the bf16 ones within one bf16 step (+1e-5 of max|b|). Both
    are also checked against the exact products by check_sublayer."""
    a, b = to_np(a) if not isinstance(a, np.ndarray) else a, to_np(b) if not isinstance(b, np.ndarray) else b
    if np.array_equal(a, b):
        return True
    if name == "dWq":
        return float(np.abs(a - b).max()) <= 1e-4 * float(np.abs(b).max())
    fa, fb = f32(a), f32(b)
    bar = bf16_ulp(np.maximum(np.abs(fa), np.abs(fb))) + 1e-5 * np.abs(fb).max()
    return bool((np.abs(fa - fb) <= bar).all())


def check_sublayer(sub, dOut, batches, threads=16, label=""):
    """sub: a metalllm_amd.sublayer.Sublayer after forward and backward (gradients zeroed first);
    dOut: the bf16 gradient at the output, numpy [B, T, C] (uint16 bits)."""
    B, T, C = sub.X.shape
    H = sub.H
    D = C // H
    g = {n: to_np(getattr(sub, n)) for n in ("X", "q", "k", "v", "o", "lse", "out", "dO", "Dv", "dQ", "dK", "dV",
                                             "dX", "dWq", "dWk", "dWv", "dWp")}
    W = {n: to_np(getattr(sub, n)) for n in ("Wq", "Wk", "Wv", "Wp")}
    dOut = np.asarray(dOut).reshape(B, T, C)
    rows = lambda a, b: np.ascontiguousarray(a.reshape(B, T, C)[b])
    heads = lambda a, b: np.ascontiguousarray(a.reshape(B, T, C)[b:b + 1].reshape(1, T, H, D))
    for b in batches:
        tag = f"{label} batch {b}"
        # forward: computeQKV, attention, projForward
        rq, rk, rv = O.computeQKV(rows(g["X"], b), W["Wq"], W["Wk"], W["Wv"], threads=threads)
        for n, r in (("q", rq), ("k", rk), ("v", rv)):
            assert bf_err(rows(g[n], b), r)[0] == 0, (tag, n)
        r_o, r_lse = O.forward(heads(g["q"], b), heads(g["k"], b), heads(g["v"], b), O.opts(threads=threads))
        lse_err = float(np.abs(g["lse"][b:b + 1] - r_lse).max())
        o_err = float(np.abs(f32(rows(g["o"], b)) - f32(r_o.reshape(T, C))).max())
        assert lse_err <= 1e-3 and o_err <= 1e-2, (tag, lse_err, o_err)
        assert bf_err(rows(g["out"], b), O.projForward(rows(g["o"], b), W["Wp"], threads=threads))[0] == 0, tag
        # backward: projBackwarddX, computeD, attention backward, computeGradDx
        assert bf_err(rows(g["dO"], b), O.projBackwarddX(rows(dOut, b), W["Wp"], threads=threads))[0] == 0, tag
        rD = O.compute_d(heads(g["dO"], b), heads(g["o"], b))
        assert np.array_equal(g["Dv"][b:b + 1], rD), tag
        rQ, rK, rV = O.backward(heads(g["dO"], b), rD, np.ascontiguousarray(g["lse"][b:b + 1]), heads(g["q"], b),
                                heads(g["k"], b), heads(g["v"], b), O.opts(threads=threads))
        errs = {n: rel_to_max(rows(g[n], b).reshape(r.shape), r) for n, r in (("dQ", rQ), ("dK", rK), ("dV", rV))}
        assert max(errs.values()) <= 2e-2, (tag, errs)
        rX = O.computeGradDx(np.zeros((T, C), np.float32), W["Wq"], W["Wk"], W["Wv"], rows(g["dQ"], b),
                             rows(g["dK"], b), rows(g["dV"], b), threads=threads)
        assert f32_err(rows(g["dX"], b), rX) <= 1e-4, tag
        print(f"  {tag}: lse {lse_err:.3g}, O {o_err:.3g}, grads rel-to-max "
              + ", ".join(f"{n} {e:.3g}" for n, e in errs.items()), flush=True)
    # weight gradients over all B*T rows, against float64 products of the GPU's operands
    R = B * T
    X64 = f32(g["X"]).reshape(R, C).astype(np.float64)
    o64 = f32(g["o"]).reshape(R, C).astype(np.float64)
    dOut64 = f32(dOut).reshape(R, C).astype(np.float64)
    dQ64 = g["dQ"].reshape(R, C).astype(np.float64)
    dK64 = f32(g["dK"]).reshape(R, C).astype(np.float64)
    dV64 = f32(g["dV"]).reshape(R, C).astype(np.float64)
    assert exact_bf_err(g["dWp"], o64.T @ dOut64) == 0, "dWp"
    assert f32_err(g["dWq"].astype(np.float64), X64.T @ dQ64) <= 1e-4, "dWq"
    assert exact_bf_err(g["dWk"], X64.T @ dK64) == 0, "dWk"
    assert exact_bf_err(g["dWv"], X64.T @ dV64) == 0, "dWv"
    print(f"  {label} weight gradients over {R} rows: within the bars", flush=True)
