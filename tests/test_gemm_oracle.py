"""Pins the CPU oracle of the sublayer GEMMs (oracle/gemm_oracle.cpp) without a GPU.

Checks chosen so that a plausible mistake fails one of them:
* exact arithmetic: small-integer bf16 operands make every product and partial sum exact in fp32,
  so the oracle must equal float64 numpy bit for bit (a wrong index, a transposed operand or a
  dropped term changes the exact result);
* random N(0,1) bf16 operands against float64 numpy, within the bound of fp32 sequential summation
  plus the destination's rounding;
* transposes against explicit transposed copies; accumulate mode (destination read once, sum
  rounded once); fp32 and bf16 destinations;
* the six named kernels against the generic GEMM composed as the reference composes them
  (attention.metal:19-53, 301-455), and against float64 numpy.
"""
import numpy as np
import pytest

import oracle as O

f32 = O.bf16_to_f32


def bf(x):
    return O.f32_to_bf16(np.asarray(x, dtype=np.float32))


def rnd(shape, seed, scale=1.0):
    return bf(np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * scale)


def ints(shape, seed, lo=-4, hi=5):
    return bf(np.random.default_rng(seed).integers(lo, hi, size=shape).astype(np.float32))


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_exact_on_small_integers(ta, tb):
    M, N, K = 19, 23, 37
    A = ints((K, M) if ta else (M, K), 1)
    B = ints((N, K) if tb else (K, N), 2)
    C = np.zeros((M, N), np.float32)
    O.gemm(A, B, C, ta=ta, tb=tb)
    a = f32(A).astype(np.float64)
    b = f32(B).astype(np.float64)
    ref = (a.T if ta else a) @ (b.T if tb else b)
    assert np.array_equal(C, ref.astype(np.float32))


def test_bf16_destination_rounds_once_and_accumulates():
    M, N, K = 8, 8, 16
    A = ints((M, K), 3)
    B = ints((K, N), 4)
    prev = bf(np.full((M, N), 0.375, np.float32))
    C = prev.copy()
    O.gemm(A, B, C, accumulate=True)
    exact = f32(A).astype(np.float64) @ f32(B).astype(np.float64) + 0.375
    assert np.array_equal(C, bf(exact.astype(np.float32)))
    C2 = prev.copy()
    O.gemm(A, B, C2, accumulate=False)
    assert np.array_equal(C2, bf((f32(A).astype(np.float64) @ f32(B).astype(np.float64)).astype(np.float32)))


def test_random_against_float64_within_summation_bound():
    M, N, K = 33, 47, 768
    A = rnd((M, K), 5)
    B = rnd((K, N), 6, 0.02)
    C = np.zeros((M, N), np.float32)
    O.gemm(A, B, C)
    a, b = f32(A).astype(np.float64), f32(B).astype(np.float64)
    ref = a @ b
    bound = K * 2.0 ** -24 * (np.abs(a) @ np.abs(b))  # sequential fp32 summation
    assert (np.abs(C - ref) <= bound + 1e-30).all()
    Cb = np.zeros((M, N), np.uint16)
    O.gemm(A, B, Cb)
    # bf16 destination: the fp32 sum rounded once (half a bf16 ulp) on top of the summation error
    assert (np.abs(f32(Cb) - ref) <= bound + np.abs(ref) * 2.0 ** -8 + 1e-30).all()


def test_fp32_operand_is_used_unrounded():
    """computeGradDx/Dw read dQ as fp32 (attention.metal:306,345): the product must use its full
    precision, not a bf16 rounding of it."""
    M, N, K = 4, 4, 8
    A = (np.arange(M * K, dtype=np.float32).reshape(M, K) + 1) * np.float32(1 + 2 ** -20)
    B = ints((K, N), 7)
    C = np.zeros((M, N), np.float32)
    O.gemm(np.ascontiguousarray(A), B, C)
    ref = (A.astype(np.float64) @ f32(B).astype(np.float64)).astype(np.float32)
    assert np.allclose(C, ref, rtol=1e-6, atol=0)
    Arnd = f32(bf(A))
    assert not np.allclose(C, (Arnd.astype(np.float64) @ f32(B).astype(np.float64)).astype(np.float32), rtol=1e-7,
                           atol=0)


def _sublayer_inputs(R=64, C=48, seed=10):
    X = rnd((R, C), seed)
    W = [rnd((C, C), seed + i, 0.02) for i in range(1, 5)]
    return X, W


def test_named_kernels_match_their_compositions():
    R, C = 64, 48
    X, (Wq, Wk, Wv, Wp) = _sublayer_inputs(R, C)
    q, k, v = O.computeQKV(X, Wq, Wk, Wv)
    for out, W in ((q, Wq), (k, Wk), (v, Wv)):
        ref = np.zeros((R, C), np.uint16)
        assert np.array_equal(out, O.gemm(X, W, ref))
    o = rnd((R, C), 20)
    out = O.projForward(o, Wp)
    assert np.array_equal(out, O.gemm(o, Wp, np.zeros((R, C), np.uint16)))
    dZ = rnd((R, C), 21)
    dWp = O.projBackwarddW(o, dZ, np.zeros((C, C), np.uint16))
    assert np.array_equal(dWp, O.gemm(o, dZ, np.zeros((C, C), np.uint16), ta=True, accumulate=True))
    dA = O.projBackwarddX(dZ, Wp)
    assert np.array_equal(dA, O.gemm(dZ, Wp, np.zeros((R, C), np.uint16), tb=True))
    dQ = np.random.default_rng(22).standard_normal((R, C)).astype(np.float32)
    dK, dV = rnd((R, C), 23), rnd((R, C), 24)
    dX = O.computeGradDx(np.zeros((R, C), np.float32), Wq, Wk, Wv, dQ, dK, dV)
    ref = np.zeros((R, C), np.float32)
    for g, W in ((dQ, Wq), (dK, Wk), (dV, Wv)):
        O.gemm(g, W, ref, tb=True, accumulate=True)
    assert np.array_equal(dX, ref)
    dQw, dKw, dVw = O.computeGradDw(X, dQ, dK, dV, np.zeros((C, C), np.float32), np.zeros((C, C), np.uint16),
                                    np.zeros((C, C), np.uint16))
    assert np.array_equal(dQw, O.gemm(X, dQ, np.zeros((C, C), np.float32), ta=True, accumulate=True))
    assert np.array_equal(dKw, O.gemm(X, dK, np.zeros((C, C), np.uint16), ta=True, accumulate=True))
    assert np.array_equal(dVw, O.gemm(X, dV, np.zeros((C, C), np.uint16), ta=True, accumulate=True))


def test_named_kernels_against_float64():
    """The reference's products, stated independently in float64 (W indexed [in][out])."""
    R, C = 64, 48
    X, (Wq, Wk, Wv, Wp) = _sublayer_inputs(R, C, 30)
    x = f32(X).astype(np.float64)
    w = [f32(W).astype(np.float64) for W in (Wq, Wk, Wv, Wp)]
    q, _, _ = O.computeQKV(X, Wq, Wk, Wv)
    assert np.allclose(f32(q), x @ w[0], rtol=2 ** -7, atol=1e-6)
    dZ = rnd((R, C), 31)
    dz = f32(dZ).astype(np.float64)
    dA = O.projBackwarddX(dZ, Wp)
    assert np.allclose(f32(dA), dz @ w[3].T, rtol=2 ** -7, atol=1e-6)
    dWp = O.projBackwarddW(X, dZ, np.zeros((C, C), np.uint16))
    assert np.allclose(f32(dWp), x.T @ dz, rtol=2 ** -7, atol=1e-4)
    dQ = np.random.default_rng(32).standard_normal((R, C)).astype(np.float32)
    dX = O.computeGradDx(np.zeros((R, C), np.float32), Wq, Wk, Wv, dQ, X, X)
    ref = dQ.astype(np.float64) @ w[0].T + x @ w[1].T + x @ w[2].T
    assert np.allclose(dX, ref, rtol=1e-5, atol=1e-6)


def test_mistake_is_caught():
    """A planted mistake (the weight of projBackwarddX not transposed) fails the float64 check:
    the check distinguishes W from W^T."""
    R, C = 64, 48
    X, (_, _, _, Wp) = _sublayer_inputs(R, C, 40)
    dz = f32(X).astype(np.float64)
    wrong = np.zeros((R, C), np.uint16)
    O.gemm(X, Wp, wrong)  # dZ.Wp instead of dZ.Wp^T
    assert not np.allclose(f32(wrong), dz @ f32(Wp).astype(np.float64).T, rtol=2 ** -7, atol=1e-6)
