"""ctypes wrapper of the CPU oracle (liboracle_attn.so, built from oracle/attn_oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker. The product (metalllm_amd/) never imports this package.

Arrays are numpy: bf16 tensors travel as uint16 bit patterns in [B, T, H, D] layout,
LSE and D as float32 [B, H, T], dQ as float32 [B, T, H, D] (accumulated into, caller zeroes).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_attn.so")
_SRC = os.path.join(_HERE, "attn_oracle.cpp")

GEMM_CHUNK16 = 0
GEMM_SEQ = 1
GEMM_MFMA = 2
PASS_SEQ8 = 0
PASS_IL4 = 1
BWD_REFERENCE = 0
BWD_FP32 = 1
DS_REFERENCE = 0
DS_FUSED = 1
DS_COUNT = 2

# Tensor ids of the seeded input generator.
TID_Q, TID_K, TID_V, TID_DO = 1, 2, 3, 4


class AttentionParams(ctypes.Structure):
    _fields_ = [("M", ctypes.c_uint32), ("N", ctypes.c_uint32), ("D", ctypes.c_uint32),
                ("NH", ctypes.c_uint32), ("B", ctypes.c_uint32)]


class OracleOpts(ctypes.Structure):
    _fields_ = [("threads", ctypes.c_int), ("b_begin", ctypes.c_int), ("b_end", ctypes.c_int),
                ("gemm_model", ctypes.c_int), ("bwd_mode", ctypes.c_int), ("d_round", ctypes.c_int),
                ("fwd_lazy", ctypes.c_float), ("ds_form", ctypes.c_int)]


def build(force: bool = False) -> str:
    """Compiles liboracle_attn.so with oracle/Makefile (gcc only, no GPU needed)."""
    if force or not os.path.exists(_LIB_PATH):
        cmd = ["make", "-C", _HERE]
        if force:
            cmd.insert(1, "-B")
        subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def build_mutant(n: int) -> str:
    """Compiles the oracle with planted mistake `n` (ORACLE_MUTANT) into oracle/_mutants/."""
    out_dir = os.path.join(_HERE, "_mutants")
    os.makedirs(out_dir, exist_ok=True)
    path = os.path.join(out_dir, f"liboracle_m{n}.so")
    if not os.path.exists(path) or os.path.getmtime(path) < os.path.getmtime(_SRC):
        subprocess.run(["g++", "-O2", "-std=c++17", "-fPIC", "-pthread", "-ffp-contract=off", f"-DORACLE_MUTANT={n}",
                        "-shared", "-o", path, _SRC], check=True)
    return path


def params(B: int, T: int, H: int, D: int) -> AttentionParams:
    return AttentionParams(T, H * D, D, H, B)


def opts(threads: int = 0, b_begin: int = 0, b_end: int = 0, gemm_model: int = GEMM_MFMA,
         bwd_mode: int = BWD_REFERENCE, d_round: int = 1, fwd_lazy: float = 0.0, ds_form: int = 0) -> OracleOpts:
    """fwd_lazy > 0 is a diagnosis mode (a lazy softmax reference point that moves only by more
    than fwd_lazy log2 units); 0 is the reference's exact running max, which the GPU forward uses.
    ds_form: DS_REFERENCE (the reference's order of dS = bf16(p*(dP - D)*scale)), DS_FUSED (the
    D = 128 GPU kernels' p*fma(dP, scale, -D*scale)) or DS_COUNT (reference order, counting the
    roundings the fused order would change: ds_flips())."""
    return OracleOpts(threads, b_begin, b_end, gemm_model, bwd_mode, d_round, fwd_lazy, ds_form)


def _check(rc: int, what: str):
    if rc != 0:
        raise ValueError(f"oracle {what} rejected the arguments (rc={rc})")


class Oracle:
    """One loaded build of the oracle library."""

    def __init__(self, path: str):
        L = ctypes.CDLL(path)
        u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        pp = ctypes.POINTER(AttentionParams)
        op = ctypes.POINTER(OracleOpts)
        L.oracle_forward.argtypes = [u16p, u16p, u16p, u16p, f32p, pp, op]
        L.oracle_forward_ex.argtypes = [u16p, u16p, u16p, u16p, f32p, f32p, pp, op]
        L.oracle_compute_d.argtypes = [u16p, u16p, f32p, pp, op]
        L.oracle_backward.argtypes = [u16p, f32p, f32p, u16p, u16p, u16p, f32p, u16p, u16p, pp, op]
        L.oracle_fill_normal_bf16.argtypes = [u16p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_float]
        L.oracle_fill_normal_bf16.restype = None
        L.oracle_dot.argtypes = [ctypes.c_float, f32p, f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.oracle_dot.restype = ctypes.c_float
        L.oracle_ds_flips.argtypes = []
        L.oracle_ds_flips.restype = ctypes.c_uint64
        self.lib = L

    def forward(self, q, k, v, o: OracleOpts | None = None):
        B, T, H, D = q.shape
        out = np.zeros_like(q)
        lse = np.zeros((B, H, T), dtype=np.float32)
        _check(self.lib.oracle_forward(q, k, v, out, lse, ctypes.byref(params(B, T, H, D)), ctypes.byref(o or opts())),
               "forward")
        return out, lse

    def forward_f32(self, q, k, v, o: OracleOpts | None = None):
        """forward() plus O*(1/l) in fp32 before its final bf16 rounding ([B, T, H, D])."""
        B, T, H, D = q.shape
        out = np.zeros_like(q)
        lse = np.zeros((B, H, T), dtype=np.float32)
        of = np.zeros((B, T, H, D), dtype=np.float32)
        _check(self.lib.oracle_forward_ex(q, k, v, out, lse, of, ctypes.byref(params(B, T, H, D)),
                                          ctypes.byref(o or opts())), "forward")
        return out, lse, of

    def compute_d(self, dO, O, o: OracleOpts | None = None):
        B, T, H, D = dO.shape
        Dv = np.zeros((B, H, T), dtype=np.float32)
        _check(self.lib.oracle_compute_d(dO, O, Dv, ctypes.byref(params(B, T, H, D)), ctypes.byref(o or opts())),
               "computeD")
        return Dv

    def backward(self, dO, Dv, lse, q, k, v, o: OracleOpts | None = None):
        B, T, H, D = q.shape
        dQ = np.zeros((B, T, H, D), dtype=np.float32)
        dK = np.zeros_like(q)
        dV = np.zeros_like(q)
        _check(self.lib.oracle_backward(dO, Dv, lse, q, k, v, dQ, dK, dV, ctypes.byref(params(B, T, H, D)),
                                        ctypes.byref(o or opts())), "backward")
        return dQ, dK, dV

    def dot(self, acc: float, a, b, model: int = GEMM_MFMA, layout: int = PASS_SEQ8) -> float:
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        return float(self.lib.oracle_dot(acc, a, b, a.size, model, layout))

    def normal_bf16(self, shape, seed: int, tensor_id: int, scale: float = 1.0) -> np.ndarray:
        out = np.empty(int(np.prod(shape)), dtype=np.uint16)
        self.lib.oracle_fill_normal_bf16(out, out.size, seed, tensor_id, scale)
        return out.reshape(shape)


_DEFAULT = None


def default() -> Oracle:
    global _DEFAULT
    if _DEFAULT is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _DEFAULT = Oracle(_LIB_PATH)
    return _DEFAULT


def lib():
    return default().lib


def normal_bf16(shape, seed: int, tensor_id: int, scale: float = 1.0) -> np.ndarray:
    """Seeded N(0,1)*scale bf16 bits; element i keyed by (seed, tensor_id, flat index i)."""
    return default().normal_bf16(shape, seed, tensor_id, scale)


def forward(q, k, v, o: OracleOpts | None = None):
    return default().forward(q, k, v, o)


def forward_f32(q, k, v, o: OracleOpts | None = None):
    return default().forward_f32(q, k, v, o)


def compute_d(dO, O, o: OracleOpts | None = None):
    return default().compute_d(dO, O, o)


def backward(dO, Dv, lse, q, k, v, o: OracleOpts | None = None):
    return default().backward(dO, Dv, lse, q, k, v, o)


def ds_flips() -> int:
    """dS values of the last backward call with ds_form=DS_COUNT whose bf16 rounding the fused
    order p*fma(dP, scale, -D*scale) changes."""
    return int(default().lib.oracle_ds_flips())


def bf16_to_f32(x: np.ndarray) -> np.ndarray:
    return (x.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (finite values)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def castFloatToBfloat(x: np.ndarray) -> np.ndarray:
    """elementwise.metal:19-28 (used at model.h:692): out[i] = bfloat(in[i]). Metal's float -> bfloat
    conversion rounds to nearest even; overflow rounds to infinity; a NaN stays a quiet NaN of the
    same sign (payload's top bits kept)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where((u & 0x7FFFFFFF) > 0x7F800000, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def _bf_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 value, as fp32 (a bfloat result of Metal bfloat arithmetic)."""
    return bf16_to_f32(f32_to_bf16(np.asarray(x, dtype=np.float32)))


def _sum32(x: np.ndarray, axis: int) -> np.ndarray:
    """An fp32 reduction, modelled order-independently: the exact sum of the fp32 terms rounded once
    to fp32 (the reference's simd_sum/threadgroup order is not specified; any order lies within the
    fp32 summation bound of this value)."""
    return np.asarray(x, dtype=np.float32).astype(np.float64).sum(axis=axis).astype(np.float32)


def residualAdd(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """elementwise.metal:7-17: out = bfloat(float(a) + float(b)) (fp32 add, one rounding)."""
    return castFloatToBfloat(bf16_to_f32(a) + bf16_to_f32(b))


def layernormForward(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float = 1e-5):
    """layernorm.metal:10-70, rows of x (bf16 bits [rows, cols]); returns (x_norm bf16, out bf16,
    stdev fp32 [rows]). fp32 arithmetic in the reference's order: mean = sum/cols, var =
    sum((x - mean)^2)/cols, std = sqrt(var + eps), rstd = 1/std, xn = (x - mean)*rstd,
    out = gamma*xn + beta (multiply and add rounded separately)."""
    xf = bf16_to_f32(x)
    cols = np.float32(xf.shape[1])
    mean = (_sum32(xf, 1) / cols).astype(np.float32)
    d = (xf - mean[:, None]).astype(np.float32)
    var = (_sum32((d * d).astype(np.float32), 1) / cols).astype(np.float32)
    sd = np.sqrt((var + np.float32(eps)).astype(np.float32)).astype(np.float32)
    rstd = (np.float32(1.0) / sd).astype(np.float32)
    xn = (d * rstd[:, None]).astype(np.float32)
    out = ((bf16_to_f32(gamma)[None, :] * xn).astype(np.float32) + bf16_to_f32(beta)[None, :]).astype(np.float32)
    return f32_to_bf16(xn), f32_to_bf16(out), sd


def layernormBackward(dZ: np.ndarray, x_norm: np.ndarray, gamma: np.ndarray, stdev: np.ndarray,
                      dgamma: np.ndarray, dbeta: np.ndarray):
    """layernorm.metal:73-127; returns (new dZ bf16, dx_norm bf16, dgamma fp32, dbeta fp32), the
    column sums added to the given dgamma/dbeta. bfloat*bfloat products are rounded to bf16
    (Metal's bfloat arithmetic): g = bf16(xn*dZ), dxn = bf16(dZ*gamma), the sum2 terms
    bf16(dxn*xn); then dZ = bf16(rdev*((dxn - sum1/cols) - xn*(sum2/cols))) with rdev = 1/stdev."""
    z = bf16_to_f32(dZ)
    x = bf16_to_f32(x_norm)
    g = bf16_to_f32(gamma)
    cols = np.float32(z.shape[1])
    dg = (np.asarray(dgamma, np.float32).astype(np.float64) + _bf_round(x * z).astype(np.float64).sum(0))
    db = (np.asarray(dbeta, np.float32).astype(np.float64) + z.astype(np.float64).sum(0))
    dxn = _bf_round(z * g[None, :])
    rs1 = (_sum32(dxn, 1) / cols).astype(np.float32)
    rs2 = (_sum32(_bf_round(dxn * x), 1) / cols).astype(np.float32)
    rdev = (np.float32(1.0) / np.asarray(stdev, np.float32)).astype(np.float32)
    t = ((dxn - rs1[:, None]).astype(np.float32) - (x * rs2[:, None]).astype(np.float32)).astype(np.float32)
    out = (rdev[:, None] * t).astype(np.float32)
    return f32_to_bf16(out), f32_to_bf16(dxn), dg.astype(np.float32), db.astype(np.float32)


# ---- sublayer GEMMs (gemm_oracle.cpp): row-major, R = B*T rows, C = NH*D features ----
T_BF16, T_F32 = 0, 1
_GEMM_BOUND = False


def _gemm_lib():
    global _GEMM_BOUND
    L = lib()
    if not _GEMM_BOUND:
        vp = ctypes.c_void_p
        i = ctypes.c_int
        L.oracle_gemm.argtypes = [i, i, i, i, i, vp, i, i, vp, i, i, vp, i, i, i, i]
        L.oracle_computeQKV.argtypes = [vp] * 7 + [i, i, i]
        L.oracle_projForward.argtypes = [vp] * 3 + [i, i, i]
        L.oracle_projBackwarddW.argtypes = [vp] * 3 + [i, i, i]
        L.oracle_projBackwarddX.argtypes = [vp] * 3 + [i, i, i]
        L.oracle_computeGradDx.argtypes = [vp] * 7 + [i, i, i]
        L.oracle_computeGradDw.argtypes = [vp] * 7 + [i, i, i]
        _GEMM_BOUND = True
    return L


def _p(x: np.ndarray):
    assert x.flags["C_CONTIGUOUS"]
    return x.ctypes.data_as(ctypes.c_void_p)


def gemm(A, B, C, ta=False, tb=False, accumulate=False, threads=0):
    """C (=|+=) op(A) . op(B), row-major; A/B/C uint16 (bf16 bits) or float32 numpy arrays."""
    M, N = C.shape
    K = A.shape[0] if ta else A.shape[1]
    t = lambda x: T_BF16 if x.dtype == np.uint16 else T_F32
    rc = _gemm_lib().oracle_gemm(int(ta), int(tb), M, N, K, _p(A), t(A), A.shape[1], _p(B), t(B), B.shape[1], _p(C),
                                 t(C), C.shape[1], int(accumulate), threads)
    _check(rc, "gemm")
    return C


def computeQKV(X, qw, kw, vw, threads=0):
    R, Cf = X.shape
    q, k, v = (np.zeros((R, Cf), np.uint16) for _ in range(3))
    _gemm_lib().oracle_computeQKV(_p(X), _p(q), _p(k), _p(v), _p(qw), _p(kw), _p(vw), R, Cf, threads)
    return q, k, v


def projForward(attn_out, proj_w, threads=0):
    R, Cf = attn_out.shape
    out = np.zeros((R, Cf), np.uint16)
    _gemm_lib().oracle_projForward(_p(attn_out), _p(proj_w), _p(out), R, Cf, threads)
    return out


def projBackwarddW(attn_out, dZ, dProjw, threads=0):
    """dProjw (bf16, accumulated into) += O^T . dZ."""
    R, Cf = attn_out.shape
    _gemm_lib().oracle_projBackwarddW(_p(attn_out), _p(dZ), _p(dProjw), R, Cf, threads)
    return dProjw


def projBackwarddX(dZ, proj_w, threads=0):
    R, Cf = dZ.shape
    dAttn = np.zeros((R, Cf), np.uint16)
    _gemm_lib().oracle_projBackwarddX(_p(dZ), _p(proj_w), _p(dAttn), R, Cf, threads)
    return dAttn


def computeGradDx(dX, qw, kw, vw, dQ, dK, dV, threads=0):
    """dX (fp32, accumulated into) += dQ.Wq^T + dK.Wk^T + dV.Wv^T (three accumulate runs)."""
    R, Cf = dX.shape
    _gemm_lib().oracle_computeGradDx(_p(dX), _p(qw), _p(kw), _p(vw), _p(dQ), _p(dK), _p(dV), R, Cf, threads)
    return dX


def computeGradDw(x, dQ, dK, dV, dQw, dKw, dVw, threads=0):
    """dQw (fp32) += X^T.dQ; dKw, dVw (bf16) += X^T.dK, X^T.dV."""
    R, Cf = x.shape
    _gemm_lib().oracle_computeGradDw(_p(x), _p(dQ), _p(dK), _p(dV), _p(dQw), _p(dKw), _p(dVw), R, Cf, threads)
    return dQw, dKw, dVw
