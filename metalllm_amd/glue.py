"""Host side of the pre-LN block's glue kernels around the attention sublayer: ctypes bindings of
residualAdd (/root/reference/elementwise.metal:7-17), castFloatToBfloat (elementwise.metal:19-28),
layernormForward and layernormBackward (/root/reference/layernorm.metal:10-127), with the
reference's buffer order and LayernormParams {rows, cols, group_size, eps} (main.cpp:89-96).

Tensors are contiguous torch tensors on the GPU: activations bf16 [rows, cols] (or [B, T, C]),
gamma/beta bf16 [cols], stdev fp32 [rows], dgamma/dbeta fp32 [cols]. No CPU fallback.
"""
from __future__ import annotations

import ctypes

from .attention import _check, _lib, _ptr, _stream


class LayernormParams(ctypes.Structure):
    """layernorm.metal:3-8: {rows, cols, group_size, eps}."""
    _fields_ = [("rows", ctypes.c_uint32), ("cols", ctypes.c_uint32), ("group_size", ctypes.c_uint32),
                ("eps", ctypes.c_float)]

    @classmethod
    def of(cls, rows: int, cols: int, eps: float = 1e-5) -> "LayernormParams":
        return cls(rows, cols, min(cols, 1024), eps)  # main.cpp:94-95


_BOUND = False


def _L():
    global _BOUND
    L = _lib()
    if not _BOUND:
        vp = ctypes.c_void_p
        lp = ctypes.POINTER(LayernormParams)
        L.residualAdd.argtypes = [vp, vp, vp, ctypes.c_uint32, vp]
        L.castFloatToBfloat.argtypes = [vp, vp, ctypes.c_uint32, vp]
        L.layernormForward.argtypes = [vp] * 6 + [lp, vp]
        L.layernormBackward.argtypes = [vp] * 7 + [lp, vp]
        for f in (L.residualAdd, L.castFloatToBfloat, L.layernormForward, L.layernormBackward):
            f.restype = ctypes.c_int
        _BOUND = True
    return L


def _rows_cols(t):
    return t.numel() // t.shape[-1], t.shape[-1]


def residualAdd(a, b, out, count=None, stream=None):
    """elementwise.metal:7-17: out = bf16(a + b) over `count` elements (all of a by default)."""
    n = a.numel() if count is None else count
    _check(_L().residualAdd(_ptr(a), _ptr(b), _ptr(out), n, _stream(stream)), "residualAdd")


def castFloatToBfloat(inp, out, count=None, stream=None):
    """elementwise.metal:19-28: out[i] = bf16(in[i]) (round to nearest even) for i < count."""
    n = inp.numel() if count is None else count
    _check(_L().castFloatToBfloat(_ptr(inp), _ptr(out), n, _stream(stream)), "castFloatToBfloat")


def layernormForward(x, x_norm, out, gamma, beta, stdev, eps: float = 1e-5, stream=None,
                     params: LayernormParams | None = None):
    """layernorm.metal:10-70: x_norm = bf16((x - mean)/stdev), out = bf16(gamma*xn + beta),
    stdev = sqrt(var + eps) per row."""
    p = params or LayernormParams.of(*_rows_cols(x), eps)
    _check(_L().layernormForward(_ptr(x), _ptr(x_norm), _ptr(out), _ptr(gamma), _ptr(beta), _ptr(stdev),
                                 ctypes.byref(p), _stream(stream)), "layernormForward")


def layernormBackward(dZ, x_norm, gamma, stdev, dgamma, dbeta, dx_norm=None, stream=None,
                      params: LayernormParams | None = None):
    """layernorm.metal:73-127, in place on dZ; dgamma/dbeta accumulated into; dx_norm (optional)
    receives bf16(dZ*gamma)."""
    p = params or LayernormParams.of(*_rows_cols(dZ))
    _check(_L().layernormBackward(_ptr(dZ), _ptr(x_norm), _ptr(gamma), _ptr(stdev), _ptr(dx_norm), _ptr(dgamma),
                                  _ptr(dbeta), ctypes.byref(p), _stream(stream)), "layernormBackward")
