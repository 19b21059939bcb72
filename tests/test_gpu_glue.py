"""GPU parity of the pre-LN glue kernels (residualAdd, layernormForward, layernormBackward;
elementwise.metal:7-17, layernorm.metal:10-127) through the C ABI against the oracle.

Bars: residualAdd and dx_norm bit-exact (one fp32 operation, one rounding, the same in both);
stdev within 2e-6 relative; x_norm and out within one bf16 ulp of the oracle's value plus the
fp32 summation bound of the row mean (cols x 2^-24 x mean|x|, times rstd, times |gamma| for out):
the GPU sums the row in another fp32 order, and where x is close to the mean, x - mean cancels,
so that difference can span many bf16 ulps of a tiny x_norm; dZ within
one bf16 ulp plus the fp32 summation slack of its two row means (2^-16 x rdev x (|dxn| + |rs1| +
|xn*rs2|)); dgamma/dbeta within 1e-5 of max |value| (fp32 sums over rows in atomic order).
"""
import numpy as np
import pytest

import oracle as O
from tests.attn_case import to_gpu, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def G():
    import metalllm_amd.glue as G
    return G


def bf(x):
    return O.f32_to_bf16(np.asarray(x, dtype=np.float32))


def ulp(v):
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def test_residual_add(gpu, G):
    import torch
    rng = np.random.default_rng(4)
    n = 1_000_005  # a count % 8 tail
    a, b = bf(rng.standard_normal(n) * 3), bf(rng.standard_normal(n))
    ta, tb = to_gpu(a, gpu), to_gpu(b, gpu)
    out = torch.empty_like(ta)
    G.residualAdd(ta, tb, out)
    G.residualAdd(ta, tb, ta)  # in place on a, as model.h:438 does
    torch.cuda.synchronize()
    ref = O.residualAdd(a, b)
    assert np.array_equal(to_np(out), ref) and np.array_equal(to_np(ta), ref)


SHAPES = [(16384, 768, 1.0), (1000, 384, 3.0), (37, 4096, 0.01), (5, 8, 1.0), (64, 2048, 1.0), (256, 520, 2.0)]


@pytest.mark.parametrize("rows,cols,scale", SHAPES)
def test_layernorm_forward_backward(gpu, G, rows, cols, scale):
    import torch
    print(f"case rows={rows} cols={cols} scale={scale}", flush=True)
    rng = np.random.default_rng(rows + cols)
    x = bf(rng.standard_normal((rows, cols)) * scale + 0.5)
    g = bf(1.0 + 0.1 * rng.standard_normal(cols))
    b = bf(0.1 * rng.standard_normal(cols))
    tx, tg, tb = to_gpu(x, gpu), to_gpu(g, gpu), to_gpu(b, gpu)
    xn = torch.empty_like(tx)
    out = torch.empty_like(tx)
    sd = torch.empty(rows, dtype=torch.float32, device=gpu)
    G.layernormForward(tx, xn, out, tg, tb, sd)
    torch.cuda.synchronize()
    r_xn, r_out, r_sd = O.layernormForward(x, g, b, 1e-5)
    g_xn, g_out, g_sd = to_np(xn), to_np(out), to_np(sd)
    assert np.abs(g_sd / r_sd - 1).max() <= 2e-6
    mean_slack = cols * 2.0 ** -24 * np.abs(O.bf16_to_f32(x)).mean(1, keepdims=True) / r_sd[:, None]
    for name, gv, rv, sl in (("x_norm", g_xn, r_xn, mean_slack),
                             ("out", g_out, r_out, mean_slack * np.abs(O.bf16_to_f32(g))[None, :])):
        d = np.abs(O.bf16_to_f32(gv) - O.bf16_to_f32(rv))
        bad = int((d > ulp(O.bf16_to_f32(rv)) + sl).sum())
        print(f"  {name}: max diff {d.max():.3g}, beyond one ulp {bad}, differing {int((gv != rv).sum())}")
        assert bad == 0
    # backward on the GPU's own forward outputs, dgamma/dbeta accumulated into nonzero values
    dZ = bf(rng.standard_normal((rows, cols)))
    dg0 = rng.standard_normal(cols).astype(np.float32)
    db0 = rng.standard_normal(cols).astype(np.float32)
    tdz, tdg, tdb = to_gpu(dZ, gpu), to_gpu(dg0, gpu), to_gpu(db0, gpu)
    dxn = torch.empty_like(tx)
    G.layernormBackward(tdz, xn, tg, sd, tdg, tdb, dx_norm=dxn)
    torch.cuda.synchronize()
    r_dz, r_dxn, r_dg, r_db = O.layernormBackward(dZ, g_xn, g, g_sd, dg0, db0)
    assert np.array_equal(to_np(dxn), r_dxn)
    gz, rz = O.bf16_to_f32(to_np(tdz)), O.bf16_to_f32(r_dz)
    xf, dxf = O.bf16_to_f32(g_xn), O.bf16_to_f32(r_dxn)
    rs1 = np.abs(dxf).mean(1, keepdims=True)
    rs2 = np.abs(dxf * xf).mean(1, keepdims=True)
    slack = 2.0 ** -16 / g_sd[:, None] * (np.abs(dxf) + rs1 + np.abs(xf) * rs2)
    d = np.abs(gz - rz)
    bad = int((d > ulp(rz) + slack).sum())
    print(f"  dZ: max diff {d.max():.3g}, beyond bar {bad}, differing {int((gz != rz).sum())}")
    assert bad == 0
    for name, gv, rv in (("dgamma", to_np(tdg), r_dg), ("dbeta", to_np(tdb), r_db)):
        e = float(np.abs(gv - rv).max() / np.abs(rv).max())
        print(f"  {name}: rel-to-max {e:.3g}")
        assert e <= 1e-5
    # without the dx_norm scratch: same dZ and sums
    tdz2, tdg2, tdb2 = to_gpu(dZ, gpu), to_gpu(dg0, gpu), to_gpu(db0, gpu)
    G.layernormBackward(tdz2, xn, tg, sd, tdg2, tdb2)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(tdz2), to_np(tdz))
