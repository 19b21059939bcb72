"""GPU parity of the sublayer GEMMs (computeQKV, projForward, projBackwarddW, projBackwarddX,
computeGradDx, computeGradDw) through the C ABI against the CPU oracle (oracle/gemm_oracle.cpp).

Bars: bf16 destinations within one bf16 ulp of the oracle's value plus 1e-5 of max|ref| (the
library sums in another order than the oracle's sequential fp32 sum, which can move a result across
a bf16 rounding boundary); fp32 destinations within 1e-4 of max|ref| (summation order, plus the
two-term bf16 split of the fp32 dQ operand, |dQ - hi - lo| <= 2^-17 |dQ|).
"""
import numpy as np
import pytest

import oracle as O
from tests.attn_case import bf16_ulp, f32, to_gpu, to_np
from tests.sublayer_check import WEIGHT_GRADS, check_sublayer, same_up_to_order

pytestmark = pytest.mark.gpu


def bf_err(gpu, ref):
    a, b = f32(gpu), f32(ref)
    d = np.abs(a - b)
    bar = bf16_ulp(b) + 1e-5 * np.abs(b).max()
    return int((d > bar).sum()), float(d.max())


def f32_err(gpu, ref):
    return float(np.abs(gpu - ref).max() / max(np.abs(ref).max(), 1e-30))


def inputs(R, C, seed):
    rng = np.random.default_rng(seed)
    X = O.f32_to_bf16(rng.standard_normal((R, C)).astype(np.float32))
    W = [O.f32_to_bf16((rng.standard_normal((C, C)) * 0.02).astype(np.float32)) for _ in range(4)]
    return X, W


@pytest.fixture(scope="module")
def S():
    import metalllm_amd.sublayer as S
    return S


@pytest.mark.parametrize("fused", [False, True])
def test_forward_gemms(gpu, S, fused):
    """fused: q_w, k_w, v_w are slices of one [3, C, C] buffer and q, k, v of one [3, R, C] buffer,
    so computeQKV runs one strided-batched product; otherwise separate buffers and three."""
    import torch
    B, T, H, C = 2, 256, 12, 768
    R = B * T
    X, (Wq, Wk, Wv, Wp) = inputs(R, C, 1)
    p = S.params_of(torch.empty((B, T, C)), H)
    tX, tq_w, tk_w, tv_w, tWp = (to_gpu(a, gpu) for a in (X, Wq, Wk, Wv, Wp))
    if fused:
        W3 = torch.stack([tq_w, tk_w, tv_w])
        tq_w, tk_w, tv_w = W3.unbind(0)
        q, k, v = torch.empty((3, R, C), dtype=torch.bfloat16, device=gpu).unbind(0)
    else:
        # a gap after each output and weight, so that they are not equally spaced
        q, k, v = (torch.empty((R + 64 * i, C), dtype=torch.bfloat16, device=gpu)[:R] for i in range(3))
        tk_w = torch.cat([tk_w, tk_w[:8]])[:C]
    P = lambda t: t.data_ptr()
    spaced = P(tk_w) - P(tq_w) == P(tv_w) - P(tk_w) and P(k) - P(q) == P(v) - P(k)
    assert spaced == fused  # the layout selects the path under test
    S.computeQKV(tX, q, k, v, tq_w, tk_w, tv_w, p)
    out = torch.empty((R, C), dtype=torch.bfloat16, device=gpu)
    S.projForward(q, tWp, out, p)
    rq, rk, rv = O.computeQKV(X, Wq, Wk, Wv, threads=16)
    for name, g, r in (("q", q, rq), ("k", k, rk), ("v", v, rv)):
        bad, mx = bf_err(to_np(g), r)
        print(f"computeQKV {name}: beyond bar {bad}, max err {mx:.3g}")
        assert bad == 0
    rout = O.projForward(to_np(q), Wp, threads=16)
    bad, mx = bf_err(to_np(out), rout)
    print(f"projForward: beyond bar {bad}, max err {mx:.3g}")
    assert bad == 0


@pytest.mark.parametrize("B,T,H,C", [(2, 256, 12, 768), (1, 384, 3, 384), (1, 256, 4, 512), (1, 320, 5, 200)])
def test_backward_gemms(gpu, S, B, T, H, C):
    """R and C multiples of 128 run the hand-written computeGradDx and computeGradDw kernels (fp32
    dQ split in registers), with 192-wide feature tiles where 192 divides C (768, 384) and 128-wide
    ones otherwise (512); the last shape runs the library path on the split dQ. For computeGradDw,
    R=512, C=768 gives 24 tiles of 128 x 192 with 8 dWq and 4 dKw/dVw row chunks each (384 items,
    dealt to the XCDs in contiguous ranges), R=384, C=384 gives 72 (not a multiple of 8 per kind:
    workgroup order) with dWq chunks of one 64-row step, and R=256, C=512 gives 16 tiles of 128 x
    128; projBackwarddW (128-wide tiles) takes 144, 27 and 32 one-weight items. All are called
    twice, so the second call accumulates into nonzero destinations."""
    import torch
    R = B * T
    X, (Wq, Wk, Wv, Wp) = inputs(R, C, 2)
    rng = np.random.default_rng(3)
    dZ = O.f32_to_bf16(rng.standard_normal((R, C)).astype(np.float32))
    dK = O.f32_to_bf16((rng.standard_normal((R, C)) * 0.1).astype(np.float32))
    dV = O.f32_to_bf16((rng.standard_normal((R, C)) * 0.1).astype(np.float32))
    dQ = (rng.standard_normal((R, C)) * 0.1).astype(np.float32)
    p = S.params_of(torch.empty((B, T, C)), H)
    g = {n: to_gpu(a, gpu) for n, a in dict(X=X, Wq=Wq, Wk=Wk, Wv=Wv, Wp=Wp, dZ=dZ, dK=dK, dV=dV, dQ=dQ).items()}
    # projBackwarddW twice: the destination is accumulated into (bf16(bf16(S) + S))
    dWp = torch.zeros((C, C), dtype=torch.bfloat16, device=gpu)
    S.projBackwarddW(g["X"], g["dZ"], dWp, p)
    S.projBackwarddW(g["X"], g["dZ"], dWp, p)
    rWp = O.projBackwarddW(X, dZ, np.zeros((C, C), np.uint16), threads=16)
    rWp = O.projBackwarddW(X, dZ, rWp, threads=16)
    bad, mx = bf_err(to_np(dWp), rWp)
    print(f"projBackwarddW x2: beyond bar {bad}, max err {mx:.3g}")
    assert bad == 0
    dA = torch.empty((R, C), dtype=torch.bfloat16, device=gpu)
    S.projBackwarddX(g["dZ"], g["Wp"], dA, p)
    bad, mx = bf_err(to_np(dA), O.projBackwarddX(dZ, Wp, threads=16))
    print(f"projBackwarddX: beyond bar {bad}, max err {mx:.3g}")
    assert bad == 0
    dX0 = (rng.standard_normal((R, C)) * 0.01).astype(np.float32)  # nonzero: accumulated into
    dX = to_gpu(dX0, gpu)
    S.computeGradDx(dX, g["Wq"], g["Wk"], g["Wv"], g["dQ"], g["dK"], g["dV"], p)
    rX = O.computeGradDx(dX0.copy(), Wq, Wk, Wv, dQ, dK, dV, threads=16)
    e = f32_err(to_np(dX), rX)
    print(f"computeGradDx: rel-to-max {e:.3g}")
    assert e <= 1e-4
    dQw = torch.zeros((C, C), dtype=torch.float32, device=gpu)
    dKw = torch.zeros((C, C), dtype=torch.bfloat16, device=gpu)
    dVw = torch.zeros((C, C), dtype=torch.bfloat16, device=gpu)
    S.computeGradDw(g["X"], g["dQ"], g["dK"], g["dV"], dQw, dKw, dVw, p)
    S.computeGradDw(g["X"], g["dQ"], g["dK"], g["dV"], dQw, dKw, dVw, p)
    rQw, rKw, rVw = O.computeGradDw(X, dQ, dK, dV, np.zeros((C, C), np.float32), np.zeros((C, C), np.uint16),
                                    np.zeros((C, C), np.uint16), threads=16)
    rQw, rKw, rVw = O.computeGradDw(X, dQ, dK, dV, rQw, rKw, rVw, threads=16)
    e = f32_err(to_np(dQw), rQw)
    print(f"computeGradDw x2 dQw: rel-to-max {e:.3g}")
    assert e <= 1e-4
    for name, t, r in (("dKw", dKw, rKw), ("dVw", dVw, rVw)):
        bad, mx = bf_err(to_np(t), r)
        print(f"computeGradDw x2 {name}: beyond bar {bad}, max err {mx:.3g}")
        assert bad == 0


def _run_chain(S, gpu, B, T, H, C, seed):
    import torch
    R = B * T
    X, (Wq, Wk, Wv, Wp) = inputs(R, C, seed)
    rng = np.random.default_rng(seed + 1)
    dOut = O.f32_to_bf16(rng.standard_normal((R, C)).astype(np.float32))
    tX = to_gpu(X.reshape(B, T, C), gpu)
    Ws = [to_gpu(w, gpu) for w in (Wq, Wk, Wv, Wp)]
    sub = S.Sublayer(tX, *Ws, H=H)
    sub.zero_grads()
    sub.forward()
    sub.backward(to_gpu(dOut.reshape(B, T, C), gpu))
    torch.cuda.synchronize()
    return sub, dOut


def test_config4_sublayer_chain(gpu, S):
    """Config 4's sublayer (C=768, H=12, D=64, T=2048) at B=1: the model.h launch sequence on the GPU;
    every stage checked against the oracle on the GPU's own inputs to that stage (attention by the
    bars of the attention parity tests)."""
    sub, dOut = _run_chain(S, gpu, 1, 2048, 12, 768, 4)
    check_sublayer(sub, dOut, batches=[0], label="config4 B=1")


def test_config4_full_size(gpu, S):
    """Config 4 at its real size, B=8, T=2048, C=768, H=12: R = 16384
    rows, so the weight gradients run the hand-written kernel's 504 items (11 dWq and 5 dKw/dVw
    row chunks per 128 x 192 tile) and the attention backward the XCD-grouped path (96 pairs).
    Row-local stages are checked on batches 0 and 7, the weight gradients over all rows; the phase
    encoder on the same inputs must give the per-call chain's results bit for bit, except the
    weight gradients, which its fused launch sums over other row chunks (same_up_to_order)."""
    import torch
    B, T, H, C = 8, 2048, 12, 768
    print(f"case config4 B={B} T={T} H={H} C={C}", flush=True)
    S.reserve(S.params_of(torch.empty((B, T, C)), H))  # scratch sized once: the calls below do not allocate
    sub, dOut = _run_chain(S, gpu, B, T, H, C, 8)
    check_sublayer(sub, dOut, batches=[0, 7], label="config4 B=8")
    enc = S.Sublayer(sub.X, sub.Wq, sub.Wk, sub.Wv, sub.Wp, H=H)
    enc.dOut.copy_(to_gpu(dOut.reshape(B, T, C), gpu))
    enc.encode(0)
    enc.encode(1)
    torch.cuda.synchronize()
    for n in ("q", "k", "v", "o", "lse", "out", "dO", "Dv", "dQ", "dK", "dV", "dX"):
        assert torch.equal(getattr(sub, n), getattr(enc, n)), n
    for n in WEIGHT_GRADS:  # the encoder's fused weight-gradient launch sums in another order
        assert same_up_to_order(n, getattr(enc, n), getattr(sub, n)), n


def test_config4_chain_at_config1_shape(gpu, S):
    """The config 4 chain at bench.py's second sublayer shape, metalLLM's own width with config 1's
    batch and length: B=128, T=256, C=384, H=6 (D=64), R = 32768 rows. The weight gradients run
    the hand-written kernel's 510 items (43 dWq and 21 dKw/dVw row chunks per 128 x 192 tile; 34
    and 17 in the encoder's four-weight launch), the attention backward the fused short-sequence
    kernel (768 pairs). Row-local stages are checked on batches 0 and 127, the weight gradients over
    all rows; the phase encoder must give the per-call chain's results bit for bit, except the
    weight gradients (same_up_to_order)."""
    import torch
    B, T, H, C = 128, 256, 6, 384
    print(f"case config4 chain B={B} T={T} H={H} C={C}", flush=True)
    S.reserve(S.params_of(torch.empty((B, T, C)), H))
    sub, dOut = _run_chain(S, gpu, B, T, H, C, 9)
    check_sublayer(sub, dOut, batches=[0, 127], label="config4 chain at c1 shape")
    enc = S.Sublayer(sub.X, sub.Wq, sub.Wk, sub.Wv, sub.Wp, H=H)
    enc.dOut.copy_(to_gpu(dOut.reshape(B, T, C), gpu))
    enc.encode(0)
    enc.encode(1)
    torch.cuda.synchronize()
    for n in ("q", "k", "v", "o", "lse", "out", "dO", "Dv", "dQ", "dK", "dV", "dX"):
        assert torch.equal(getattr(sub, n), getattr(enc, n)), n
    for n in WEIGHT_GRADS:
        assert same_up_to_order(n, getattr(enc, n), getattr(sub, n)), n
