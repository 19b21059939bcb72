"""GPU parity: the HIP kernels through the C ABI against the CPU oracle on identical seeded inputs.

Bars: LSE within 1e-3; O within 1e-2 max-abs, except elements whose
bf16 spacing exceeds 1e-2 (|O| >= 2), where the bar is one bf16 ulp of the oracle's value;
dQ/dK/dV within 2e-2 max-abs relative to max |grad|; computeD bit-exact (same inputs, same
summation order); causal-mask and index logic exact (row 0 of O equals row 0 of V bit for bit).
Both backward entry points are checked: flashAttentionBackward and flashAttentionBackwardWorkspace
(the stored-dS path); their dK/dV must also be identical to each other, their dQ equal within
1e-5 of max |dQ| (fp32 summation order).
"""
import ctypes
import os

import numpy as np
import pytest

import oracle as O
from tests.attn_case import (f32, gpu_backward, gpu_compute_d, gpu_forward, make_inputs, out_error, rel_to_max,
                             to_gpu, to_np)

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def check_case(gpu, B, T, H, D, s, seed, b_end=0, threads=0):
    """Forward, computeD and backward against the oracle; the oracle runs batches [0, b_end)."""
    print(f"case B={B} T={T} H={H} D={D} qk_scale={s} seed={seed} oracle-batches={b_end or B}", flush=True)
    q, k, v, g = make_inputs(B, T, H, D, seed, s)
    nb = b_end or B
    sl = lambda x: np.ascontiguousarray(x[:nb])
    r_out, r_lse = O.forward(sl(q), sl(k), sl(v), O.opts(threads=threads))
    ref = {"out": r_out, "lse": r_lse}
    out, lse = gpu_forward(q, k, v, gpu)
    lse_err = float(np.abs(lse[:nb] - ref["lse"]).max())
    o_max, o_bad, o_over = out_error(out[:nb], ref["out"])
    print(f"  fwd: lse max err {lse_err:.3g}, O max err {o_max:.3g}, O beyond bar {o_bad}, O > 1e-2 {o_over}")
    assert np.isfinite(lse).all() and lse_err <= 1e-3
    assert o_bad == 0
    # computeD on the GPU's own O; the oracle on the same O must agree bit for bit
    Dfull = gpu_compute_d(g, out, gpu)
    Dr = O.compute_d(sl(g), sl(out))
    assert np.array_equal(Dfull[:nb], Dr), f"computeD differs: {np.abs(Dfull[:nb] - Dr).max()}"
    # backward alone: both sides get the GPU's lse and D
    rQ, rK, rV = O.backward(sl(g), Dr, np.ascontiguousarray(lse[:nb]), sl(q), sl(k), sl(v), O.opts(threads=threads))
    res = []
    for ws in (False, True):
        dQ, dK, dV = gpu_backward(g, Dfull, lse, q, k, v, gpu, workspace=ws)
        errs = {n: rel_to_max(x[:nb], r) for n, x, r in (("dQ", dQ, rQ), ("dK", dK, rK), ("dV", dV, rV))}
        print(f"  bwd{' (workspace)' if ws else ''} rel-to-max:", {n: f"{e:.3g}" for n, e in errs.items()}, flush=True)
        for n, e in errs.items():
            assert e <= 2e-2, n
        res.append((dQ, dK, dV))
    (q0, k0, v0), (q1, k1, v1) = res
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
    assert np.abs(q0 - q1).max() <= 1e-5 * np.abs(q0).max()
    return out, lse


CASES = [
    # (B, T, H, D, qk_scale, seed)
    (16, 256, 6, 64, 1.0, 11),    # config 0: the reference default shape
    (2, 512, 2, 128, 1.0, 12),    # D=128
    (1, 1024, 12, 64, 1.5, 13),   # config 2 slice: peaky rows
    (1, 192, 3, 128, 1.5, 14),    # T not a multiple of 128/256, odd head count
    (1, 64, 1, 64, 1.0, 15),      # a single tile
    (3, 320, 1, 64, 1.0, 16),     # 5 tiles, B*H not a multiple of 8
    (4, 448, 2, 128, 1.0, 17),    # 8 pairs: XCD-affine two-tile dQ ring (T < 512), 7 tiles
    (2, 576, 4, 128, 1.0, 18),    # 8 pairs: XCD-affine four-tile dQ ring, last item 1 of 4 tiles
]


@pytest.mark.parametrize("B,T,H,D,s,seed", CASES)
def test_forward_backward_parity(gpu, B, T, H, D, s, seed):
    check_case(gpu, B, T, H, D, s, seed)


def test_config1_slice_equals_config0(gpu):
    """Config 1 (B=128) on the GPU; its first 16 batches are config 0's inputs bit for bit, and are
    checked against the oracle."""
    out, lse = check_case(gpu, 128, 256, 6, 64, 1.0, 21, b_end=16)
    q0, k0, v0, _ = make_inputs(16, 256, 6, 64, 21)
    out0, lse0 = gpu_forward(q0, k0, v0, gpu)
    assert np.array_equal(out[:16], out0) and np.array_equal(lse[:16], lse0)


def test_config2_peaky_slice(gpu):
    """Config 2 (B=32, H=12, T=1024, D=64, Q/K x1.5): two batches checked against the oracle."""
    check_case(gpu, 32, 1024, 12, 64, 1.5, 22, b_end=2)


def test_config3_slice(gpu):
    """Config 3 (B=16, H=16, T=4096, D=128) at B=1: all 16 heads of batch 0 against the oracle."""
    check_case(gpu, 1, 4096, 16, 128, 1.0, 23)


def test_config3_full_size_properties(gpu):
    """Config 3 at full size: row 0 of every head equals V row 0 bit for bit (causal index logic),
    LSE finite, forward and backward deterministic across runs, sum over keys of dV equal to the
    sum over queries of dO (rows of P sum to 1); the workspace backward gives identical dK/dV and
    dQ within fp32 summation order."""
    import torch
    import metalllm_amd as M
    B, T, H, D = 16, 4096, 16, 128
    dev = gpu
    g_ = torch.Generator(device=dev)
    g_.manual_seed(7)
    mk = lambda: torch.randn((B, T, H, D), generator=g_, device=dev).to(torch.bfloat16)
    q, k, v, dO = mk(), mk(), mk(), mk()
    out1, lse1 = M.attention_forward(q, k, v)
    out2, lse2 = M.attention_forward(q, k, v)
    assert torch.equal(out1, out2) and torch.equal(lse1, lse2)
    assert torch.equal(out1[:, 0], v[:, 0])
    assert torch.isfinite(lse1).all()
    dQ1, dK1, dV1, Dv = M.attention_backward(dO, q, k, v, out1, lse1)
    dQ2, dK2, dV2, _ = M.attention_backward(dO, q, k, v, out1, lse1)
    assert torch.equal(dK1, dK2) and torch.equal(dV1, dV2) and torch.equal(dQ1, dQ2)
    ws = torch.empty((M.workspace_bytes(B, T, H, D),), dtype=torch.uint8, device=dev)
    dQ3, dK3, dV3 = torch.empty_like(dQ1), torch.empty_like(dK1), torch.empty_like(dV1)
    M.flashAttentionBackwardWorkspace(dO, Dv, lse1, q, k, v, dQ3, dK3, dV3, ws)
    assert torch.equal(dK1, dK3) and torch.equal(dV1, dV3)
    assert (dQ1 - dQ3).abs().max().item() <= 1e-5 * dQ1.abs().max().item()
    del ws
    sdv = dV1.float().sum(1)
    sdo = dO.float().sum(1)
    assert ((sdv - sdo).abs().max() / sdo.abs().max()).item() < 3e-2


def test_mfma_model_on_random_tiles(gpu):
    """The oracle's matrix-core model reproduces v_mfma_f32_32x32x16_bf16 bit for bit on random
    tiles: N(0,1) operands, scaled operands, mixed magnitudes, and nonzero accumulators."""
    import torch
    lib = ctypes.CDLL(os.path.join(HERE, "golden", "libmfma_probe.so"))
    lib.mfma_probe_run.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int, ctypes.c_void_p]
    rng = np.random.default_rng(11)
    n = 48
    scale = np.exp(rng.uniform(-6, 6, size=(n, 64, 8)))
    a = O.f32_to_bf16((rng.standard_normal((n, 64, 8)) * scale).astype(np.float32))
    b = O.f32_to_bf16(rng.standard_normal((n, 64, 8)).astype(np.float32))
    c = (rng.standard_normal((n, 64, 16)) * rng.choice([0, 1e-3, 1, 30], size=(n, 1, 1))).astype(np.float32)
    ta, tb, tc = to_gpu(a, gpu), to_gpu(b, gpu), to_gpu(c, gpu)
    assert lib.mfma_probe_run(ta.data_ptr(), tb.data_ptr(), tc.data_ptr(), n, torch.cuda.current_stream().cuda_stream) == 0
    res = to_np(tc)
    orc = O.default()
    A = f32(a)
    Bm = f32(b)
    bad = 0
    for t in range(n):
        Am = np.zeros((32, 16), np.float32)
        Bt = np.zeros((32, 16), np.float32)  # [n][k]
        for l in range(64):
            Am[l % 32, 8 * (l // 32):8 * (l // 32) + 8] = A[t, l]
            Bt[l % 32, 8 * (l // 32):8 * (l // 32) + 8] = Bm[t, l]
        for l in range(64):
            for r in range(16):
                m = 8 * (r // 4) + 4 * (l // 32) + r % 4
                nn = l % 32
                ref = orc.dot(float(c[t, l, r]), Am[m], Bt[nn], O.GEMM_MFMA, O.PASS_SEQ8)
                bad += np.float32(ref) != res[t, l, r]
    assert bad == 0, f"{bad} of {n * 1024} results differ from the model"


def test_backward_writes_gradients_in_full(gpu):
    """ABI contract: dQ, dK and dV are written in full (stale contents ignored: the result equals
    the reference's accumulation into zeroed buffers), by both entry points, and a workspace's
    stale contents do not matter either."""
    import torch
    import metalllm_amd as M
    for T in (256, 192):
        q, k, v, g = make_inputs(1, T, 2, 64, 31)
        tq, tk, tv, tg = (to_gpu(x, gpu) for x in (q, k, v, g))
        out, lse = M.attention_forward(tq, tk, tv)
        Dv = torch.empty((1, 2, T), dtype=torch.float32, device=gpu)
        M.computeD(tg, out, Dv)
        ws = torch.full((M.workspace_bytes(1, T, 2, 64),), 0x7F, dtype=torch.uint8, device=gpu)
        res = []
        for fill in (0.0, 7.0, float("nan")):
            for use_ws in (False, True):
                dQ = torch.full((1, T, 2, 64), fill, dtype=torch.float32, device=gpu)
                dK = torch.full_like(tq, fill)
                dV = torch.full_like(tq, -fill)
                if use_ws:
                    M.flashAttentionBackwardWorkspace(tg, Dv, lse, tq, tk, tv, dQ, dK, dV, ws)
                else:
                    M.flashAttentionBackward(tg, Dv, lse, tq, tk, tv, dQ, dK, dV)
                res.append((use_ws, dQ, dK, dV))
        for use_ws, dQ, dK, dV in res:
            ref = res[0] if not use_ws else res[1]
            assert torch.isfinite(dQ).all() and torch.equal(dQ, ref[1])
            assert torch.equal(dK, res[0][2]) and torch.equal(dV, res[0][3])


def test_backward_parts_equal_flash_attention_backward(gpu):
    """The bench hook: part 0 (dK/dV kernel) then part 1 (dQ kernel) is flashAttentionBackward, and
    part 2 then part 3 is flashAttentionBackwardWorkspace, bit for bit."""
    import torch
    import metalllm_amd as M
    q, k, v, g = make_inputs(2, 512, 3, 128, 41)
    tq, tk, tv, tg = (to_gpu(x, gpu) for x in (q, k, v, g))
    out, lse = M.attention_forward(tq, tk, tv)
    Dv = torch.empty((2, 3, 512), dtype=torch.float32, device=gpu)
    M.computeD(tg, out, Dv)
    ws = torch.empty((M.workspace_bytes(2, 512, 3, 128),), dtype=torch.uint8, device=gpu)
    for first in (0, 2):
        res = []
        for split in (False, True):
            dQ = torch.empty((2, 512, 3, 128), dtype=torch.float32, device=gpu)
            dK = torch.empty_like(tq)
            dV = torch.empty_like(tq)
            if split:
                M.backward_part(first, tg, Dv, lse, tq, tk, tv, dQ, dK, dV, workspace=ws)
                M.backward_part(first + 1, tg, Dv, lse, tq, tk, tv, dQ, dK, dV, workspace=ws)
            elif first == 0:
                M.flashAttentionBackward(tg, Dv, lse, tq, tk, tv, dQ, dK, dV)
            else:
                M.flashAttentionBackwardWorkspace(tg, Dv, lse, tq, tk, tv, dQ, dK, dV, ws)
            res.append((dQ, dK, dV))
        for a, b in zip(*res):
            assert torch.equal(a, b)
