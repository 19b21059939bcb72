"""Host side of the attention sublayer around the attention core: ctypes bindings of the six GEMM
entry points of libmetalllm_attn.so (computeQKV, projForward, projBackwarddW, projBackwarddX,
computeGradDx, computeGradDw; /root/reference/attention.metal:19-53, 301-455), of the dX handoff
castFloatToBfloat (elementwise.metal:19-28, model.h:692), and of the phase encoder: the sublayer's
forward and backward chains in the order /root/reference/model.h:446-482 and :621-693 encode them,
enqueued eagerly (metalllmSublayerEncode) or recorded once as a HIP graph per phase and replayed
(metalllmSublayerGraph*), the MI355X form of model.h's one command buffer per phase.

Tensors are torch tensors on the GPU, contiguous: activations [B, T, C] (or [R, C]) with C = H*D,
weights [C, C] indexed [input feature][output feature]. No CPU fallback: every product runs on
the device through the library.
"""
from __future__ import annotations

import ctypes

from .attention import (AttentionParams, _check, _lib, _ptr, _stream, backward_part, computeD, flashAttentionForward,
                        workspace_bytes)
from .glue import castFloatToBfloat  # noqa: F401  (the dX handoff, model.h:692)

_BOUND = False


def _L():
    global _BOUND
    L = _lib()
    if not _BOUND:
        vp = ctypes.c_void_p
        pp = ctypes.POINTER(AttentionParams)
        L.computeQKV.argtypes = [vp] * 7 + [pp, vp]
        L.projForward.argtypes = [vp] * 3 + [pp, vp]
        L.projBackwarddW.argtypes = [vp] * 3 + [pp, vp]
        L.projBackwarddX.argtypes = [vp] * 3 + [pp, vp]
        L.computeGradDx.argtypes = [vp] * 7 + [pp, vp]
        L.computeGradDw.argtypes = [vp] * 7 + [pp, vp]
        bp = ctypes.POINTER(SublayerBuffers)
        L.metalllmSublayerEncode.argtypes = [ctypes.c_int, bp, pp, vp]
        L.metalllmSublayerGraphCreate.argtypes = [ctypes.c_int, bp, pp, ctypes.POINTER(vp)]
        L.metalllmSublayerGraphLaunch.argtypes = [vp, vp]
        L.metalllmSublayerGraphDestroy.argtypes = [vp]
        L.metalllmSublayerReserve.argtypes = [pp]
        for f in (L.metalllmSublayerReserve, L.computeQKV, L.projForward, L.projBackwarddW, L.projBackwarddX, L.computeGradDx, L.computeGradDw,
                  L.metalllmSublayerEncode, L.metalllmSublayerGraphCreate,
                  L.metalllmSublayerGraphLaunch, L.metalllmSublayerGraphDestroy):
            f.restype = ctypes.c_int
        _BOUND = True
    return L


class SublayerBuffers(ctypes.Structure):
    """metalllmSublayerBuffers: the sublayer's device buffers (model.h:236-277), field order as in
    include/metalllm_attn.h."""
    FIELDS = ("X", "q_w", "k_w", "v_w", "proj_w", "q", "k", "v", "attn_out", "l", "out", "dOut", "dAttn", "Dsum", "dQ",
              "dK", "dV", "dX", "dQw", "dKw", "dVw", "dProjw", "dX_bf16", "hidden", "ln_gamma", "ln_beta", "ln_xnorm",
              "ln_stdev", "ln_dgamma", "ln_dbeta", "residual", "dStream")
    _fields_ = [(n, ctypes.c_void_p) for n in FIELDS] + [("ln_eps", ctypes.c_float)]


def params_of(x, H: int) -> AttentionParams:
    """AttentionParams of an activation [B, T, C] (or [R, C], taken as B = 1) with H heads."""
    if x.dim() == 3:
        B, T, C = x.shape
    else:
        (T, C), B = x.shape, 1
    return AttentionParams.of(B, T, H, C // H)


def computeQKV(X, q, k, v, q_w, k_w, v_w, p: AttentionParams, stream=None):
    """attention.metal:19-53: q, k, v = X.q_w, X.k_w, X.v_w (bf16)."""
    _check(_L().computeQKV(_ptr(X), _ptr(q), _ptr(k), _ptr(v), _ptr(q_w), _ptr(k_w), _ptr(v_w), ctypes.byref(p),
                           _stream(stream)), "computeQKV")


def projForward(attn_out, proj_w, out, p: AttentionParams, stream=None):
    """attention.metal:385-405: out = attn_out.proj_w (bf16)."""
    _check(_L().projForward(_ptr(attn_out), _ptr(proj_w), _ptr(out), ctypes.byref(p), _stream(stream)), "projForward")


def projBackwarddW(attn_out, dZ, dProjw, p: AttentionParams, stream=None):
    """attention.metal:407-430: dProjw += attn_out^T.dZ (bf16, accumulated)."""
    _check(_L().projBackwarddW(_ptr(attn_out), _ptr(dZ), _ptr(dProjw), ctypes.byref(p), _stream(stream)),
           "projBackwarddW")


def projBackwarddX(dZ, proj_w, dAttn, p: AttentionParams, stream=None):
    """attention.metal:432-455: dAttn = dZ.proj_w^T (bf16)."""
    _check(_L().projBackwarddX(_ptr(dZ), _ptr(proj_w), _ptr(dAttn), ctypes.byref(p), _stream(stream)),
           "projBackwarddX")


def computeGradDx(dX, qw, kw, vw, dQ, dK, dV, p: AttentionParams, stream=None):
    """attention.metal:301-341: dX += dQ.qw^T + dK.kw^T + dV.vw^T (fp32, accumulated)."""
    _check(_L().computeGradDx(_ptr(dX), _ptr(qw), _ptr(kw), _ptr(vw), _ptr(dQ), _ptr(dK), _ptr(dV), ctypes.byref(p),
                              _stream(stream)), "computeGradDx")


def computeGradDw(x, dQ, dK, dV, dQw, dKw, dVw, p: AttentionParams, stream=None):
    """attention.metal:343-383: dQw += x^T.dQ (fp32); dKw, dVw += x^T.dK, x^T.dV (bf16); accumulated."""
    _check(_L().computeGradDw(_ptr(x), _ptr(dQ), _ptr(dK), _ptr(dV), _ptr(dQw), _ptr(dKw), _ptr(dVw),
                              ctypes.byref(p), _stream(stream)), "computeGradDw")


def reserve(p: AttentionParams):
    """metalllmSublayerReserve: size the current device's scratch for shape p once (synchronises
    the device if it grows), so later GEMM and encoder calls up to that shape never allocate."""
    _check(_L().metalllmSublayerReserve(ctypes.byref(p)), "metalllmSublayerReserve")


def encode_phase(phase: int, bufs: SublayerBuffers, p: AttentionParams, stream=None):
    """metalllmSublayerEncode: enqueue phase 0 (forward) or 1 (backward) eagerly."""
    _check(_L().metalllmSublayerEncode(phase, ctypes.byref(bufs), ctypes.byref(p), _stream(stream)),
           "metalllmSublayerEncode")


class PhaseGraph:
    """One phase recorded as a HIP graph (metalllmSublayerGraphCreate); launch() replays it."""

    def __init__(self, phase: int, bufs: SublayerBuffers, p: AttentionParams):
        self._g = ctypes.c_void_p()
        self._L = _L()
        _check(self._L.metalllmSublayerGraphCreate(phase, ctypes.byref(bufs), ctypes.byref(p), ctypes.byref(self._g)),
               "metalllmSublayerGraphCreate")

    def launch(self, stream=None):
        _check(self._L.metalllmSublayerGraphLaunch(self._g, _stream(stream)), "metalllmSublayerGraphLaunch")

    def close(self):
        if self._g:
            import torch
            torch.cuda.synchronize()
            _check(self._L.metalllmSublayerGraphDestroy(self._g), "metalllmSublayerGraphDestroy")
            self._g = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Sublayer:
    """Buffers and launch sequence of one attention sublayer (pre-LN block, without the layernorm
    and residual glue), mirroring model.h: forward computeQKV -> flashAttentionForward ->
    projForward (model.h:446-482); backward projBackwarddW, projBackwarddX, computeD,
    flashAttentionBackward, computeGradDx, computeGradDw (model.h:621-690), with the gradient
    buffers zeroed first as model.h:549-555 does."""

    def __init__(self, X, Wq, Wk, Wv, Wp, H: int, hidden=None, ln_gamma=None, ln_beta=None, ln_eps: float = 1e-5):
        """X: the sublayer input [B, T, C]. With `hidden` (and ln_gamma, ln_beta) the phase encoder
        runs the block's attention half: X is then allocated here and written by ln1(hidden)."""
        import torch
        if hidden is not None:
            X = torch.empty_like(hidden)
        self.X, self.Wq, self.Wk, self.Wv, self.Wp, self.H = X, Wq, Wk, Wv, Wp, H
        B, T, C = X.shape
        self.p = params_of(X, H)
        D = C // H
        dev = X.device
        bf = lambda: torch.empty((B, T, C), dtype=torch.bfloat16, device=dev)
        # q, k, v as three equal slices of one buffer: with a fused [3, C, C] weight (equally spaced
        # q_w, k_w, v_w) computeQKV runs one batched product
        self.qkv = torch.empty((3, B, T, C), dtype=torch.bfloat16, device=dev)
        self.q, self.k, self.v = self.qkv.unbind(0)
        self.o, self.out = bf(), bf()
        self.lse = torch.empty((B, H, T), dtype=torch.float32, device=dev)
        self.dO, self.dK, self.dV = bf(), bf(), bf()
        self.Dv = torch.empty((B, H, T), dtype=torch.float32, device=dev)
        self.dQ = torch.empty((B, T, C), dtype=torch.float32, device=dev)
        self.ws = torch.empty((workspace_bytes(B, T, H, D),), dtype=torch.uint8, device=dev)
        self.dX = torch.zeros((B, T, C), dtype=torch.float32, device=dev)
        self.dWq = torch.zeros((C, C), dtype=torch.float32, device=dev)
        self.dWk = torch.zeros((C, C), dtype=torch.bfloat16, device=dev)
        self.dWv = torch.zeros((C, C), dtype=torch.bfloat16, device=dev)
        self.dWp = torch.zeros((C, C), dtype=torch.bfloat16, device=dev)
        self.dOut = bf()      # the phase encoder's input gradient buffer (model.h's dBranch)
        self.dXb = bf()       # bf16(dX), the handoff to the layernorm backward (model.h:692)
        self.D = D
        self.graphs = None
        self.hidden, self.ln_gamma, self.ln_beta, self.ln_eps = hidden, ln_gamma, ln_beta, ln_eps
        if hidden is not None:
            self.ln_xnorm, self.residual, self.dStream = bf(), bf(), bf()
            self.ln_stdev = torch.empty((B * T,), dtype=torch.float32, device=dev)
            self.ln_dgamma = torch.empty((C,), dtype=torch.float32, device=dev)
            self.ln_dbeta = torch.empty((C,), dtype=torch.float32, device=dev)

    def buffers(self, cast: bool = True) -> SublayerBuffers:
        """The struct of device pointers; cast=False leaves dX_bf16 NULL (no dX handoff)."""
        b = SublayerBuffers()
        t = dict(X=self.X, q_w=self.Wq, k_w=self.Wk, v_w=self.Wv, proj_w=self.Wp, q=self.q, k=self.k, v=self.v,
                 attn_out=self.o, l=self.lse, out=self.out, dOut=self.dOut, dAttn=self.dO, Dsum=self.Dv, dQ=self.dQ,
                 dK=self.dK, dV=self.dV, dX=self.dX, dQw=self.dWq, dKw=self.dWk, dVw=self.dWv, dProjw=self.dWp,
                 dX_bf16=self.dXb)
        if not cast:
            t["dX_bf16"] = None
        blk = ("hidden", "ln_gamma", "ln_beta", "ln_xnorm", "ln_stdev", "ln_dgamma", "ln_dbeta", "residual", "dStream")
        for n in blk:
            t[n] = getattr(self, n) if self.hidden is not None else None
        for n in SublayerBuffers.FIELDS:
            setattr(b, n, _ptr(t[n]).value if t[n] is not None else None)
        b.ln_eps = self.ln_eps
        return b

    def encode(self, phase: int, stream=None):
        """One phase through the native encoder (eager launches). Phase 1 reads self.dOut and
        zeroes the accumulated gradients first, as model.h:549-555 does."""
        encode_phase(phase, self.buffers(), self.p, stream)

    def capture(self):
        """Records both phases as HIP graphs on the current buffers."""
        b = self.buffers()
        self.graphs = (PhaseGraph(0, b, self.p), PhaseGraph(1, b, self.p))
        return self.graphs

    def replay(self, phase: int, stream=None):
        self.graphs[phase].launch(stream)

    def close(self):
        if self.graphs:
            for g in self.graphs:
                g.close()
            self.graphs = None

    def forward(self, stream=None):
        p = self.p
        computeQKV(self.X, self.q, self.k, self.v, self.Wq, self.Wk, self.Wv, p, stream)
        flashAttentionForward(self.q, self.k, self.v, self.o, self.lse, stream, p)
        projForward(self.o, self.Wp, self.out, p, stream)
        return self.out

    def zero_grads(self):
        for t in (self.dX, self.dWq, self.dWk, self.dWv, self.dWp):
            t.zero_()

    def backward(self, dOut, stream=None, parts=None):
        """dOut: gradient at the sublayer output [B, T, C] bf16. `parts`, if given, is a list of
        (name, callable) hooks run between launches (the bench records events there)."""
        p = self.p
        mark = (lambda name: parts(name)) if parts else (lambda name: None)
        projBackwarddW(self.o, dOut, self.dWp, p, stream)
        projBackwarddX(dOut, self.Wp, self.dO, p, stream)
        mark("proj")
        computeD(self.dO, self.o, self.Dv, stream, p)
        # flashAttentionBackwardWorkspace, as its two kernels (the bench times them separately)
        backward_part(2, self.dO, self.Dv, self.lse, self.q, self.k, self.v, self.dQ, self.dK, self.dV, stream, p,
                      workspace=self.ws)
        backward_part(3, self.dO, self.Dv, self.lse, self.q, self.k, self.v, self.dQ, self.dK, self.dV, stream, p,
                      workspace=self.ws)
        mark("attention")
        computeGradDx(self.dX, self.Wq, self.Wk, self.Wv, self.dQ, self.dK, self.dV, p, stream)
        computeGradDw(self.X, self.dQ, self.dK, self.dV, self.dWq, self.dWk, self.dWv, p, stream)
        mark("grads")
        return self.dX
