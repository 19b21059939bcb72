"""Host side of the attention hot path: ctypes bindings of libmetalllm_attn.so.

The three entry points mirror the reference's kernels and their dispatch sites
(/root/reference/attention.metal:56-299, /root/reference/model.h:459-473,639-665): same names,
same buffer order, caller-owned buffers; dQ, dK and dV written in full (the reference's
accumulation into zeroed buffers gives the same result), and a faster backward variant with a
caller-provided device workspace (flashAttentionBackwardWorkspace). PyTorch only
provides device memory and the stream; every computation happens in the HIP kernels. There is
no CPU fallback: if the library is missing, or a tensor is not on a GPU, these functions raise.

Tensors: q, k, v, out, dO, dK, dV are torch.bfloat16 [B, T, H, D]; lse and D are torch.float32
[B, H, T]; dQ is torch.float32 [B, T, H, D]. All contiguous.
"""
from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libmetalllm_attn.so")

OK = 0
ERRORS = {
    -1: "E_NULL", -2: "E_SEQLEN", -3: "E_HEADDIM", -4: "E_LAYOUT", -5: "E_SIZE", -6: "E_ALIGN", -7: "E_LAUNCH",
    -8: "E_LIBRARY", -9: "E_CAPTURE",
}
EXPORTED = ("flashAttentionForward", "computeD", "flashAttentionBackward", "metalllmAttnBackwardPart",
            "metalllmAttnErrorString", "metalllmAttnWorkMap", "computeQKV", "projForward", "projBackwarddW",
            "projBackwarddX", "computeGradDx", "computeGradDw", "castFloatToBfloat", "metalllmSublayerEncode",
            "flashAttentionBackwardWorkspace", "metalllmAttnBackwardWorkspaceSize", "residualAdd",
            "layernormForward", "layernormBackward",
            "metalllmSublayerGraphCreate", "metalllmSublayerGraphLaunch", "metalllmSublayerGraphDestroy",
            "metalllmSublayerReserve", "flashAttentionBackwardNoAlloc", "metalllmAttnForwardItems")
NOALLOC_SCRATCH_BYTES = 64 << 20  # METALLLM_ATTN_NOALLOC_SCRATCH_BYTES


class AttentionParams(ctypes.Structure):
    """attention.metal:7-12 {M, N, D, NH} with B appended."""
    _fields_ = [("M", ctypes.c_uint32), ("N", ctypes.c_uint32), ("D", ctypes.c_uint32),
                ("NH", ctypes.c_uint32), ("B", ctypes.c_uint32)]

    @classmethod
    def of(cls, B: int, T: int, H: int, D: int) -> "AttentionParams":
        return cls(T, H * D, D, H, B)


class AttentionError(RuntimeError):
    def __init__(self, code: int, what: str):
        self.code = code
        super().__init__(f"{what}: {ERRORS.get(code, code)} ({_lib().metalllmAttnErrorString(code).decode()})")


_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m metalllm_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        vp = ctypes.c_void_p
        pp = ctypes.POINTER(AttentionParams)
        L.flashAttentionForward.argtypes = [vp, vp, vp, vp, vp, pp, vp]
        L.computeD.argtypes = [vp, vp, vp, pp, vp]
        L.flashAttentionBackward.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, pp, vp]
        u64 = ctypes.c_uint64
        L.metalllmAttnBackwardPart.argtypes = [ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, u64, pp, vp]
        L.flashAttentionBackwardWorkspace.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, u64, pp, vp]
        L.metalllmAttnBackwardWorkspaceSize.argtypes = [pp, ctypes.POINTER(u64)]
        L.flashAttentionBackwardNoAlloc.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, pp, vp]
        for f in (L.flashAttentionForward, L.computeD, L.flashAttentionBackward, L.metalllmAttnBackwardPart,
                  L.flashAttentionBackwardWorkspace, L.metalllmAttnBackwardWorkspaceSize,
                  L.flashAttentionBackwardNoAlloc):
            f.restype = ctypes.c_int
        L.metalllmAttnErrorString.argtypes = [ctypes.c_int]
        L.metalllmAttnErrorString.restype = ctypes.c_char_p
        L.metalllmAttnWorkMap.argtypes = [ctypes.c_int, pp, ctypes.c_void_p, ctypes.c_int32]
        L.metalllmAttnWorkMap.restype = ctypes.c_int
        L.metalllmAttnForwardItems.argtypes = [pp, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32]
        L.metalllmAttnForwardItems.restype = ctypes.c_int
        _LIB = L
    return _LIB


def library():
    """The loaded ctypes library (loads it on first use)."""
    return _lib()


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("tensor must live on the GPU")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _shape(q):
    B, T, H, D = q.shape
    return AttentionParams.of(B, T, H, D)


def _check(rc: int, what: str):
    if rc != OK:
        raise AttentionError(rc, what)


def flashAttentionForward(q, k, v, out, l, stream=None, params: AttentionParams | None = None):
    """attention.metal:56-164. Writes out (bf16) and l = logsumexp (fp32 [B,H,T])."""
    p = params or _shape(q)
    _check(_lib().flashAttentionForward(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(l), ctypes.byref(p),
                                        _stream(stream)), "flashAttentionForward")


def computeD(dO, O, D, stream=None, params: AttentionParams | None = None):
    """attention.metal:166-195. D = bf16(rowsum(bf16(dO*O))), fp32 [B,H,T]."""
    p = params or _shape(dO)
    _check(_lib().computeD(_ptr(dO), _ptr(O), _ptr(D), ctypes.byref(p), _stream(stream)), "computeD")


def flashAttentionBackward(dZ, d, l, q, k, v, dQ, dK, dV, stream=None, params: AttentionParams | None = None):
    """attention.metal:198-299. dQ += grad (fp32, accumulated into as the reference's atomics do: zero it
    first for the plain gradient); dK, dV = grads (bf16), written in full."""
    p = params or _shape(q)
    _check(_lib().flashAttentionBackward(_ptr(dZ), _ptr(d), _ptr(l), _ptr(q), _ptr(k), _ptr(v), _ptr(dQ), _ptr(dK),
                                         _ptr(dV), ctypes.byref(p), _stream(stream)), "flashAttentionBackward")


def workspace_bytes(B: int, T: int, H: int, D: int) -> int:
    """Device workspace flashAttentionBackwardWorkspace needs (bytes)."""
    n = ctypes.c_uint64()
    _check(_lib().metalllmAttnBackwardWorkspaceSize(ctypes.byref(AttentionParams.of(B, T, H, D)), ctypes.byref(n)),
           "metalllmAttnBackwardWorkspaceSize")
    return n.value


def _ws(workspace):
    if workspace is None:
        return None, 0
    return _ptr(workspace), workspace.numel() * workspace.element_size()


def flashAttentionBackwardWorkspace(dZ, d, l, q, k, v, dQ, dK, dV, workspace, stream=None,
                                    params: AttentionParams | None = None):
    """flashAttentionBackward with a device workspace (a tensor of at least workspace_bytes bytes)
    holding the stored dS tiles; dK, dV identical. dQ is written in full (= the gradient), equal to
    what flashAttentionBackward adds into a zeroed dQ up to fp32 summation order."""
    p = params or _shape(q)
    wp, wn = _ws(workspace)
    _check(_lib().flashAttentionBackwardWorkspace(_ptr(dZ), _ptr(d), _ptr(l), _ptr(q), _ptr(k), _ptr(v), _ptr(dQ),
                                                  _ptr(dK), _ptr(dV), wp, wn, ctypes.byref(p), _stream(stream)),
           "flashAttentionBackwardWorkspace")


def flashAttentionBackwardNoAlloc(dZ, d, l, q, k, v, dQ, dK, dV, stream=None, params: AttentionParams | None = None):
    """flashAttentionBackwardWorkspace with the dS tiles in the library's fixed 64 MiB per-device
    array: allocates nothing; calls overlapping on one GPU race; shapes whose tiles exceed the
    array raise (E_SIZE)."""
    p = params or _shape(q)
    _check(_lib().flashAttentionBackwardNoAlloc(_ptr(dZ), _ptr(d), _ptr(l), _ptr(q), _ptr(k), _ptr(v), _ptr(dQ),
                                                _ptr(dK), _ptr(dV), ctypes.byref(p), _stream(stream)),
           "flashAttentionBackwardNoAlloc")


def backward_part(part: int, dZ, d, l, q, k, v, dQ, dK, dV, stream=None, params: AttentionParams | None = None,
                  workspace=None):
    """One kernel of the backward entry points (0: dK/dV, 1: dQ recomputing the softmax = the two
    kernels of flashAttentionBackward; 2: dK/dV storing dS into `workspace`, 3: dQ from the stored
    dS = flashAttentionBackwardWorkspace); the bench times them separately."""
    p = params or _shape(q)
    wp, wn = _ws(workspace)
    _check(_lib().metalllmAttnBackwardPart(part, _ptr(dZ), _ptr(d), _ptr(l), _ptr(q), _ptr(k), _ptr(v), _ptr(dQ),
                                           _ptr(dK), _ptr(dV), wp, wn, ctypes.byref(p), _stream(stream)),
           "metalllmAttnBackwardPart")


def attention_forward(q, k, v, stream=None):
    """Allocating convenience wrapper: returns (out, lse)."""
    import torch
    B, T, H, D = q.shape
    out = torch.empty_like(q)
    lse = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
    flashAttentionForward(q, k, v, out, lse, stream)
    return out, lse


def attention_backward(dO, q, k, v, out, lse, stream=None):
    """The reference's backward sequence (model.h:639-665 dispatches): computeD,
    flashAttentionBackward into a zeroed dQ (model.h:549). Returns (dQ fp32, dK, dV, D)."""
    import torch
    B, T, H, D = q.shape
    dQ = torch.zeros((B, T, H, D), dtype=torch.float32, device=q.device)
    dK = torch.empty_like(q)
    dV = torch.empty_like(q)
    Dv = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
    computeD(dO, out, Dv, stream)
    flashAttentionBackward(dO, Dv, lse, q, k, v, dQ, dK, dV, stream)
    return dQ, dK, dV, Dv


def forward_items(B: int, T: int, H: int, D: int, grid: int):
    """(workgroup, pair, block) of every item of the persistent forward on `grid` workgroups, each
    workgroup's items in the order it runs them."""
    import numpy as np
    p = AttentionParams.of(B, T, H, D)
    n = _lib().metalllmAttnForwardItems(ctypes.byref(p), grid, None, 0)
    _check(min(n, 0), "metalllmAttnForwardItems")
    out = np.zeros((n, 3), dtype=np.int32)
    _check(min(_lib().metalllmAttnForwardItems(ctypes.byref(p), grid, out.ctypes.data_as(ctypes.c_void_p), n), 0),
           "metalllmAttnForwardItems")
    return out


def work_map(kind: int, B: int, T: int, H: int, D: int):
    """(pair, block) owned by each workgroup id of the forward (0), dK/dV (1) or dQ (2) grid."""
    import numpy as np
    p = AttentionParams.of(B, T, H, D)
    n = _lib().metalllmAttnWorkMap(kind, ctypes.byref(p), None, 0)
    _check(min(n, 0), "metalllmAttnWorkMap")
    out = np.zeros((n, 2), dtype=np.int32)
    _check(min(_lib().metalllmAttnWorkMap(kind, ctypes.byref(p), out.ctypes.data_as(ctypes.c_void_p), n), 0),
           "metalllmAttnWorkMap")
    return out
