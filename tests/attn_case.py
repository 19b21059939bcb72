"""Shared helpers: seeded inputs from the oracle's generator, oracle runs, GPU runs, error metrics."""
from __future__ import annotations

import numpy as np

import oracle as O


def make_inputs(B, T, H, D, seed=1, qk_scale=1.0):
    q = O.normal_bf16((B, T, H, D), seed, O.TID_Q, qk_scale)
    k = O.normal_bf16((B, T, H, D), seed, O.TID_K, qk_scale)
    v = O.normal_bf16((B, T, H, D), seed, O.TID_V)
    g = O.normal_bf16((B, T, H, D), seed, O.TID_DO)
    return q, k, v, g


def oracle_all(q, k, v, g, **kw):
    o = O.opts(**kw)
    out, lse = O.forward(q, k, v, o)
    Dv = O.compute_d(g, out, o)
    dQ, dK, dV = O.backward(g, Dv, lse, q, k, v, o)
    return dict(out=out, lse=lse, D=Dv, dQ=dQ, dK=dK, dV=dV)


def to_gpu(x, dev):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    if x.dtype == np.uint16:
        t = t.view(torch.bfloat16)
    return t.to(dev)


def to_np(t):
    import torch
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def gpu_forward(q, k, v, dev):
    import metalllm_amd as M
    out, lse = M.attention_forward(to_gpu(q, dev), to_gpu(k, dev), to_gpu(v, dev))
    return to_np(out), to_np(lse)


def gpu_backward(g, Dv, lse, q, k, v, dev, workspace=False):
    """flashAttentionBackward (or, with workspace, flashAttentionBackwardWorkspace) alone on given
    D / lse. dK and dV start filled with NaN (both entry points write them in full); dQ starts at
    zero for flashAttentionBackward, which adds into it as the reference does, and at NaN for the
    workspace variant, which writes it in full."""
    import torch
    import metalllm_amd as M
    tq, tk, tv, tg = (to_gpu(x, dev) for x in (q, k, v, g))
    dQ = torch.full(q.shape, float("nan") if workspace else 0.0, dtype=torch.float32, device=dev)
    dK = torch.full_like(tq, float("nan"))
    dV = torch.full_like(tq, float("nan"))
    if workspace:
        B, T, H, D = q.shape
        ws = torch.full((M.workspace_bytes(B, T, H, D),), 0xFF, dtype=torch.uint8, device=dev)
        M.flashAttentionBackwardWorkspace(tg, to_gpu(Dv, dev), to_gpu(lse, dev), tq, tk, tv, dQ, dK, dV, ws)
    else:
        M.flashAttentionBackward(tg, to_gpu(Dv, dev), to_gpu(lse, dev), tq, tk, tv, dQ, dK, dV)
    return to_np(dQ), to_np(dK), to_np(dV)


def gpu_compute_d(g, out, dev):
    import torch
    import metalllm_amd as M
    B, T, H, D = g.shape
    Dv = torch.empty((B, H, T), dtype=torch.float32, device=dev)
    M.computeD(to_gpu(g, dev), to_gpu(out, dev), Dv)
    return to_np(Dv)


def f32(x):
    return O.bf16_to_f32(x) if x.dtype == np.uint16 else x.astype(np.float32)


def bf16_ulp(x):
    """Spacing of bf16 values at |x| (normal range)."""
    ax = np.maximum(np.abs(x), np.float32(2.0 ** -126))
    e = np.floor(np.log2(ax))
    return np.exp2(e - 7).astype(np.float32)


def out_error(out_gpu, out_ref):
    """Max abs error of O, and the count of elements beyond max(1e-2, 1 bf16 ulp of the reference)."""
    a, b = f32(out_gpu), f32(out_ref)
    d = np.abs(a - b)
    bar = np.maximum(np.float32(1e-2), bf16_ulp(b))
    return float(d.max()), int((d > bar).sum()), int((d > 1e-2).sum())


def out_exceptions(out_gpu, out_ref_f32, bar=1e-2):
    """Elements of O beyond the north_star's 1e-2 max-abs bar, each classified. An element whose
    magnitude is at least 2 has a bf16 spacing of 1/64 > 1e-2, so two correct roundings of values
    a hair apart can differ by one spacing: such an element is an output rounding flip when the
    GPU's bf16 value is within one spacing of the oracle's unrounded fp32 value (O*(1/l) before its
    final rounding, attention.metal:161). Returns (flips, unexplained) as lists of flat indices."""
    a = f32(out_gpu).ravel()
    x = np.asarray(out_ref_f32, dtype=np.float32).ravel()
    ref = f32(O.f32_to_bf16(x))
    over = np.nonzero(np.abs(a - ref) > bar)[0]
    ulp = bf16_ulp(x[over])
    is_flip = (np.abs(x[over]) >= 2.0) & (np.abs(a[over] - x[over]) <= ulp)
    return over[is_flip].tolist(), over[~is_flip].tolist()


def rel_to_max(x, ref):
    a, b = f32(x), f32(ref)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))
