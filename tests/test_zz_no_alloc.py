"""flashAttentionBackwardNoAlloc (no counterpart in the reference; for callers that cannot
allocate) through the C ABI against flashAttentionBackwardWorkspace, the entry point whose kernels
it shares: dQ, dK and dV bit-identical, on two calls in a row, the second with a smaller input
(the fixed per-device dS array keeps the first call's tiles; every tile the second call reads it
writes first). Outputs start filled with NaN: the entry point writes them in full."""
import ctypes

import numpy as np
import pytest

from tests.attn_case import make_inputs, to_gpu

pytestmark = pytest.mark.gpu


def _run(gpu, B, T, H, D, seed):
    import torch
    import metalllm_amd as M
    print(f"case B={B} T={T} H={H} D={D} seed={seed}", flush=True)
    q, k, v, g = (to_gpu(x, gpu) for x in make_inputs(B, T, H, D, seed))
    out, lse = M.attention_forward(q, k, v)
    Dv = torch.empty((B, H, T), dtype=torch.float32, device=gpu)
    M.computeD(g, out, Dv)
    ws = torch.empty((M.workspace_bytes(B, T, H, D),), dtype=torch.uint8, device=gpu)
    ref = [torch.full((B, T, H, D), float("nan"), dtype=torch.float32, device=gpu),
           torch.full_like(q, float("nan")), torch.full_like(q, float("nan"))]
    M.flashAttentionBackwardWorkspace(g, Dv, lse, q, k, v, *ref, ws)
    got = [torch.full_like(t, float("nan")) for t in ref]
    lib = M.library()
    p = M.AttentionParams.of(B, T, H, D)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = lib.flashAttentionBackwardNoAlloc(ptr(g), ptr(Dv), ptr(lse), ptr(q), ptr(k), ptr(v), *(ptr(t) for t in got),
                                           ctypes.byref(p), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, rc
    torch.cuda.synchronize()
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def test_no_alloc_backward_matches_workspace_backward(gpu):
    # D = 128 stores dS tiles in the array: 53.5 MB of them (near its 64 MiB), then a smaller input
    _run(gpu, 4, 1024, 12, 128, 61)
    _run(gpu, 2, 512, 4, 128, 62)
    # D = 64 stores no tiles (T <= 256: the fused short backward; longer: the recomputing kernels):
    # accepted beyond the array's nominal size (120 MiB and 104 MiB of tiles here)
    _run(gpu, 256, 256, 6, 64, 63)
    _run(gpu, 8, 2048, 3, 64, 64)
    import metalllm_amd as M
    assert M.workspace_bytes(8, 2048, 3, 64) > M.attention.NOALLOC_SCRATCH_BYTES
    with pytest.raises(M.AttentionError):  # D = 128 tiles beyond the array: rejected before the device
        import torch
        x = torch.empty((8, 1024, 12, 128), dtype=torch.bfloat16, device=gpu)
        d = torch.empty((8, 12, 1024), dtype=torch.float32, device=gpu)
        dq = torch.empty((8, 1024, 12, 128), dtype=torch.float32, device=gpu)
        M.flashAttentionBackwardNoAlloc(x, d, d, x, x, x, dq, x, x)
