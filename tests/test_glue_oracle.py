"""Pins the oracle of the dX handoff castFloatToBfloat (elementwise.metal:19-28) without a GPU:
known answers for round-to-nearest-even (ties to even both ways, carries into the exponent,
overflow to infinity, subnormals, signed zero) and, on random and special inputs, agreement with
torch's own float32 -> bfloat16 conversion on the CPU (a library routine that rounds to nearest
even)."""
import numpy as np
import torch

import oracle as O


def bits(vals):
    return np.array(vals, dtype=np.uint32).view(np.float32)


def test_known_answers():
    x = bits([0x3F800000,   # 1.0
              0x3F808000,   # 1 + 2^-8: a tie, rounds down to the even 0x3F80
              0x3F818000,   # 1 + 3*2^-8: a tie, rounds up to the even 0x3F82
              0x3F808001,   # just above the tie: up
              0x3F7FFFFF,   # carry into the exponent: 1.0
              0x7F7FFFFF,   # largest finite: overflows to +inf
              0xFF7FFFFF,   # to -inf
              0x7F800000, 0xFF800000,  # infinities stay
              0x80000000, 0x00000000,  # signed zeros
              0x00018000,   # subnormal tie between 0x0001 and 0x0002: up to the even 0x0002
              0x7F800001,   # signalling NaN: quiet NaN, same sign
              0xFFC12345])  # quiet negative NaN keeps sign and top payload bits
    want = [0x3F80, 0x3F80, 0x3F82, 0x3F81, 0x3F80, 0x7F80, 0xFF80, 0x7F80, 0xFF80, 0x8000, 0x0000, 0x0002,
            0x7FC0, 0xFFC1]
    assert O.castFloatToBfloat(x).tolist() == want


def test_matches_torch_conversion():
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(100_000).astype(np.float32),
        (rng.standard_normal(10_000) * 1e-40).astype(np.float32),          # subnormals
        rng.integers(0, 2 ** 32, size=100_000, dtype=np.uint64).astype(np.uint32).view(np.float32),  # every class
    ])
    got = O.castFloatToBfloat(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    g = got[nan]
    assert ((g & 0x7F80) == 0x7F80).all() and ((g & 0x7F) != 0).all()  # NaN stays NaN
    assert np.array_equal(g >> 15, (x[nan].view(np.uint32) >> 31).astype(np.uint16))  # sign kept


def test_planted_truncation_is_caught():
    """Truncation instead of rounding (a plausible mistake) fails the known answers."""
    x = bits([0x3F808001, 0x3F7FFFFF])
    trunc = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert trunc.tolist() != O.castFloatToBfloat(x).tolist()


# ---- residualAdd, layernormForward / layernormBackward ----

def _bf(x):
    return O.f32_to_bf16(np.asarray(x, dtype=np.float32))


def test_residual_add_matches_torch_bf16_add():
    rng = np.random.default_rng(3)
    a = _bf(rng.standard_normal(50_001) * 4)
    b = _bf(rng.standard_normal(50_001))
    ta = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    tb = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    ref = (ta + tb).view(torch.int16).numpy().view(np.uint16)  # fp32 add, rounded once to bf16
    assert np.array_equal(O.residualAdd(a, b), ref)


def _ln_inputs(rows, cols, seed, scale=1.0, shift=0.0):
    rng = np.random.default_rng(seed)
    x = _bf(rng.standard_normal((rows, cols)) * scale + shift)
    g = _bf(1.0 + 0.1 * rng.standard_normal(cols))
    b = _bf(0.1 * rng.standard_normal(cols))
    return x, g, b


def _torch_ln(x, g, b, eps, dZ=None):
    """float64 layer norm on the same bf16 inputs (and its input gradient for dZ)."""
    xt = torch.from_numpy(O.bf16_to_f32(x).astype(np.float64)).requires_grad_(True)
    gt = torch.from_numpy(O.bf16_to_f32(g).astype(np.float64))
    bt = torch.from_numpy(O.bf16_to_f32(b).astype(np.float64))
    y = torch.nn.functional.layer_norm(xt, (x.shape[1],), gt, bt, eps)
    xn = (xt - xt.mean(1, keepdim=True)) / torch.sqrt(xt.var(1, unbiased=False, keepdim=True) + eps)
    if dZ is None:
        return xn.detach().numpy(), y.detach().numpy(), None
    y.backward(torch.from_numpy(O.bf16_to_f32(dZ).astype(np.float64)))
    return xn.detach().numpy(), y.detach().numpy(), xt.grad.numpy()


def _ulp(v):
    """bf16 spacing at |v| (fp32 values), with the subnormal floor."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def test_layernorm_forward_against_float64():
    for (rows, cols, scale, shift) in ((64, 768, 1.0, 0.0), (32, 384, 3.0, 5.0), (8, 4096, 0.01, 0.0)):
        x, g, b = _ln_inputs(rows, cols, rows + cols, scale, shift)
        xn, out, sd = O.layernormForward(x, g, b, 1e-5)
        r_xn, r_out, _ = _torch_ln(x, g, b, 1e-5)
        xf = O.bf16_to_f32(x).astype(np.float64)
        r_sd = np.sqrt(xf.var(1) + 1e-5)
        assert np.abs(sd / r_sd - 1).max() < 1e-5
        # one bf16 rounding of a value carrying fp32-level error
        assert (np.abs(O.bf16_to_f32(xn) - r_xn) <= _ulp(r_xn) * 0.5 + 1e-5 * (1 + np.abs(r_xn))).all()
        assert (np.abs(O.bf16_to_f32(out) - r_out) <= _ulp(r_out) * 0.5 + 1e-4 * (1 + np.abs(r_out))).all()


def test_layernorm_forward_closed_forms():
    # a constant row: mean c, variance 0, stdev sqrt(eps), x_norm 0, out = beta
    x = _bf(np.full((1, 64), 2.5))
    g, b = _bf(np.full(64, 1.5)), _bf(np.linspace(-1, 1, 64))
    xn, out, sd = O.layernormForward(x, g, b, 1e-5)
    assert sd[0] == np.float32(np.sqrt(np.float32(1e-5)))
    assert (xn == 0).all() and np.array_equal(out[0], b)
    # alternating +-1: mean 0, variance 1, x_norm = +-1/sqrt(1 + eps) -> bf16(+-1)
    x = _bf(np.tile([1.0, -1.0], 32)[None, :])
    xn, out, sd = O.layernormForward(x, _bf(np.ones(64)), _bf(np.zeros(64)), 1e-5)
    assert abs(float(sd[0]) - np.sqrt(1 + 1e-5)) < 1e-7
    assert np.array_equal(xn, _bf(np.tile([1.0, -1.0], 32)[None, :]))


def test_layernorm_backward_against_float64_autograd():
    for (rows, cols) in ((64, 768), (16, 384), (4, 4096)):
        x, g, b = _ln_inputs(rows, cols, 7 + cols)
        dZ = _bf(np.random.default_rng(cols).standard_normal((rows, cols)))
        xn, _, sd = O.layernormForward(x, g, b, 1e-5)
        dg0 = np.random.default_rng(1).standard_normal(cols).astype(np.float32)
        db0 = np.random.default_rng(2).standard_normal(cols).astype(np.float32)
        new_dZ, dxn, dg, db = O.layernormBackward(dZ, xn, g, sd, dg0, db0)
        r_xn, _, r_dx = _torch_ln(x, g, b, 1e-5, dZ)
        z = O.bf16_to_f32(dZ).astype(np.float64)
        assert np.abs(O.bf16_to_f32(new_dZ) - r_dx).max() <= 2e-2 * np.abs(r_dx).max()
        r_dg = dg0 + (r_xn * z).sum(0)
        r_db = db0 + z.sum(0)
        assert np.abs(dg - r_dg).max() <= 1e-2 * np.abs(r_dg).max()
        assert np.abs(db - r_db).max() <= 1e-5 * np.abs(r_db).max()
        assert np.array_equal(dxn, _bf(O.bf16_to_f32(dZ) * O.bf16_to_f32(g)[None, :]))


def test_layernorm_backward_planted_mistakes_are_caught():
    """The float64-autograd check rejects a dropped mean(dxn) term and a dropped x_norm*mean term."""
    rows, cols = 32, 384
    x, g, b = _ln_inputs(rows, cols, 99, 1.0, 0.5)
    dZ = _bf(np.random.default_rng(98).standard_normal((rows, cols)) + 0.3)
    xn, _, sd = O.layernormForward(x, g, b, 1e-5)
    _, _, r_dx = _torch_ln(x, g, b, 1e-5, dZ)
    z, xf, gf = O.bf16_to_f32(dZ), O.bf16_to_f32(xn), O.bf16_to_f32(g)
    dxn = z * gf[None, :]
    rdev = 1.0 / sd[:, None]
    no_mean = rdev * (dxn - xf * (dxn * xf).mean(1, keepdims=True))
    no_proj = rdev * (dxn - dxn.mean(1, keepdims=True))
    for wrong in (no_mean, no_proj):
        assert np.abs(wrong - r_dx).max() > 2e-2 * np.abs(r_dx).max()
