"""C ABI checks that need no GPU: the library loads, exports what include/metalllm_attn.h declares,
and rejects invalid arguments before touching the device."""
import ctypes
import os
import re

import pytest

import metalllm_amd as M
from metalllm_amd.attention import AttentionParams, EXPORTED

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "metalllm_attn.h")).read()
    return set(re.findall(r"^(?:int|const char\*)\s+(\w+)\(", text, flags=re.M))


def test_library_exports_every_declared_symbol():
    lib = M.library()
    names = declared_functions()
    assert names == set(EXPORTED)
    for n in names:
        assert hasattr(lib, n), n


BAD = [
    (dict(M=0), -2), (dict(M=100), -2), (dict(M=65), -2),
    (dict(D=32), -3), (dict(D=96), -3), (dict(D=256), -3),
    (dict(N=383), -4), (dict(NH=0, N=0), -4), (dict(B=0), -4),
    (dict(B=1 << 12, M=1 << 16), -5),
]


@pytest.mark.parametrize("change,code", BAD)
def test_invalid_shapes_rejected_without_device(change, code):
    lib = M.library()
    f = dict(M=256, N=384, D=64, NH=6, B=1)
    f.update(change)
    p = AttentionParams(f["M"], f["N"], f["D"], f["NH"], f["B"])
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    assert lib.flashAttentionForward(fake, fake, fake, fake, fake, ctypes.byref(p), None) == code
    assert lib.computeD(fake, fake, fake, ctypes.byref(p), None) == code
    assert lib.flashAttentionBackward(fake, fake, fake, fake, fake, fake, fake, fake, fake, ctypes.byref(p), None) == code
    for part in (0, 1, 2, 3):
        assert lib.metalllmAttnBackwardPart(part, fake, fake, fake, fake, fake, fake, fake, fake, fake, fake, 1 << 40,
                                            ctypes.byref(p), None) == code
    assert lib.flashAttentionBackwardWorkspace(fake, fake, fake, fake, fake, fake, fake, fake, fake, fake, 1 << 40,
                                               ctypes.byref(p), None) == code
    n = ctypes.c_uint64()
    assert lib.metalllmAttnBackwardWorkspaceSize(ctypes.byref(p), ctypes.byref(n)) == code


def test_null_and_alignment_rejected():
    lib = M.library()
    p = AttentionParams(256, 384, 64, 6, 1)
    ok = ctypes.c_void_p(1 << 20)
    assert lib.flashAttentionForward(ok, ok, None, ok, ok, ctypes.byref(p), None) == -1
    assert lib.computeD(ok, None, ok, ctypes.byref(p), None) == -1
    assert lib.flashAttentionBackward(ok, ok, ok, ok, ok, ok, None, ok, ok, ctypes.byref(p), None) == -1
    assert lib.flashAttentionBackwardWorkspace(ok, ok, ok, ok, ok, ok, None, ok, ok, ok, 1 << 40, ctypes.byref(p),
                                               None) == -1
    assert lib.flashAttentionForward(ok, ok, ok, ok, ok, None, None) == -1
    bad = ctypes.c_void_p((1 << 20) + 2)
    assert lib.flashAttentionForward(ok, ok, bad, ok, ok, ctypes.byref(p), None) == -6
    assert lib.computeD(ok, ok, bad, ctypes.byref(p), None) == -6


def test_backward_part_rejects_unknown_part():
    lib = M.library()
    p = AttentionParams(256, 384, 64, 6, 1)
    fake = ctypes.c_void_p(16)
    for part in (-1, 4, 7):
        assert lib.metalllmAttnBackwardPart(part, fake, fake, fake, fake, fake, fake, fake, fake, fake, None, 0,
                                            ctypes.byref(p), None) == -4


def test_workspace_size_and_validation():
    """metalllmAttnBackwardWorkspaceSize is B*NH*(M/64)(M/64+1)/2 * 8192 bytes (64-bit, past 2^32 at
    the target shape); the workspace entry point and parts 2/3 reject a NULL, misaligned or short
    workspace before touching the device; parts 0/1 ignore it."""
    lib = M.library()
    n = ctypes.c_uint64()
    for (B, T, H, D) in ((1, 64, 1, 64), (2, 192, 3, 128), (16, 4096, 16, 128), (128, 256, 6, 64)):
        p = AttentionParams(T, H * D, D, H, B)
        assert lib.metalllmAttnBackwardWorkspaceSize(ctypes.byref(p), ctypes.byref(n)) == 0
        t = T // 64
        assert n.value == B * H * t * (t + 1) // 2 * 8192
    assert M.workspace_bytes(16, 4096, 16, 128) == 16 * 16 * 64 * 65 // 2 * 8192 > 1 << 32
    p = AttentionParams(256, 384, 64, 6, 1)
    assert lib.metalllmAttnBackwardWorkspaceSize(ctypes.byref(p), None) == -1
    assert lib.metalllmAttnBackwardWorkspaceSize(ctypes.byref(p), ctypes.byref(n)) == 0
    need = n.value
    ok = ctypes.c_void_p(1 << 20)
    args = [ok] * 9
    f = lib.flashAttentionBackwardWorkspace
    assert f(*args, None, need, ctypes.byref(p), None) == -1
    assert f(*args, ctypes.c_void_p((1 << 20) + 8), need, ctypes.byref(p), None) == -6
    assert f(*args, ok, need - 1, ctypes.byref(p), None) == -5
    for part in (2, 3):
        assert lib.metalllmAttnBackwardPart(part, *args, None, need, ctypes.byref(p), None) == -1
        assert lib.metalllmAttnBackwardPart(part, *args, ok, need - 16, ctypes.byref(p), None) == -5


def test_error_strings():
    lib = M.library()
    for code in range(-9, 1):
        assert lib.metalllmAttnErrorString(code)
    assert lib.metalllmAttnErrorString(-9) != lib.metalllmAttnErrorString(-100)


def test_no_alloc_backward_validates_before_device():
    """flashAttentionBackwardNoAlloc rejects shapes whose dS tiles exceed its fixed array (at
    D = 128; at D = 64 the workspace entry point stores no tiles), bad shapes, NULL and misaligned
    pointers before touching the device."""
    lib = M.library()
    f = lib.flashAttentionBackwardNoAlloc
    ok = ctypes.c_void_p(1 << 20)
    fits = AttentionParams.of(4, 1024, 12, 128)     # 53.5 MB of dS tiles
    too_big = AttentionParams.of(8, 1024, 12, 128)  # 107 MB
    assert M.workspace_bytes(4, 1024, 12, 128) <= M.attention.NOALLOC_SCRATCH_BYTES < M.workspace_bytes(8, 1024, 12, 128)
    assert f(*([ok] * 9), ctypes.byref(too_big), None) == -5
    # D = 64 stores no dS tiles: config 1 (60 MiB of nominal tiles, the fused short backward), a
    # batch 8x larger (480 MiB), config 2 (792 MiB) and config 4's attention (T = 2048, 816 MiB; the
    # recomputing kernels) pass the size step and stop at the NULL pointer
    over = ((1024, 256, 6, 64), (32, 1024, 12, 64), (8, 2048, 12, 64))
    assert all(M.workspace_bytes(*shape) > M.attention.NOALLOC_SCRATCH_BYTES for shape in over)
    for shape in ((128, 256, 6, 64),) + over:
        assert f(*([ok] * 8), None, ctypes.byref(AttentionParams.of(*shape)), None) == -1
    assert f(*([ok] * 9), ctypes.byref(AttentionParams.of(1, 100, 1, 64)), None) == -2
    assert f(*([ok] * 8), None, ctypes.byref(fits), None) == -1
    assert f(*([ok] * 8), ctypes.c_void_p((1 << 20) + 2), ctypes.byref(fits), None) == -6


def test_sublayer_reserve_validates_before_device():
    """metalllmSublayerReserve rejects shapes the sublayer cannot run before touching the device."""
    lib = M.library()
    lib.metalllmSublayerReserve.argtypes = [ctypes.POINTER(AttentionParams)]
    assert lib.metalllmSublayerReserve(None) == -1
    for fields, code in (((0, 768, 64, 12, 8), -2), ((2048, 767, 64, 12, 8), -4), ((2048, 1536, 128, 8, 8), -4),
                         ((2048, 96 * 8, 96, 8, 8), -3), ((2000, 768, 64, 12, 8), -2)):
        assert lib.metalllmSublayerReserve(ctypes.byref(AttentionParams(*fields))) == code, fields


GEMM_ARGS = {  # entry point -> number of tensor pointers before the params pointer
    "computeQKV": 7, "projForward": 3, "projBackwarddW": 3, "projBackwarddX": 3, "computeGradDx": 7, "computeGradDw": 7,
}


@pytest.mark.parametrize("name", sorted(GEMM_ARGS))
def test_sublayer_gemms_validate_before_device(name):
    """The sublayer GEMM entry points reject bad shapes, NULL and misaligned pointers without a
    device call (M = 0, N != NH*D, oversized tensors; D is free: these are plain GEMMs)."""
    lib = M.library()
    f = getattr(lib, name)
    n = GEMM_ARGS[name]
    ok = ctypes.c_void_p(1 << 20)
    good = dict(M=256, N=384, D=64, NH=6, B=1)
    for change, code in ((dict(M=0), -2), (dict(N=383), -4), (dict(NH=0, N=0), -4), (dict(B=0), -4),
                         (dict(B=1 << 12, M=1 << 16), -5)):
        g = dict(good)
        g.update(change)
        p = AttentionParams(g["M"], g["N"], g["D"], g["NH"], g["B"])
        assert f(*([ok] * n), ctypes.byref(p), None) == code, (name, change)
    p = AttentionParams(256, 384, 64, 6, 1)
    assert f(*([ok] * (n - 1)), None, ctypes.byref(p), None) == -1
    assert f(*([ok] * (n - 1)), ctypes.c_void_p((1 << 20) + 4), ctypes.byref(p), None) == -6
    assert f(*([ok] * n), None, None) == -1


def test_cast_validates_before_device():
    lib = M.library()
    f = lib.castFloatToBfloat
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p]
    ok = ctypes.c_void_p(1 << 20)
    assert f(None, None, 0, None) == 0  # count 0: nothing to do
    assert f(None, ok, 16, None) == -1
    assert f(ok, None, 16, None) == -1
    assert f(ctypes.c_void_p((1 << 20) + 8), ok, 16, None) == -6
    assert f(ok, ctypes.c_void_p((1 << 20) + 2), 16, None) == -6


def test_sublayer_buffers_struct_matches_header():
    """The ctypes struct's field order is the header's."""
    from metalllm_amd.sublayer import SublayerBuffers
    text = open(os.path.join(ROOT, "include", "metalllm_attn.h")).read()
    body = text[text.index("typedef struct metalllmSublayerBuffers {"):text.index("} metalllmSublayerBuffers;")]
    names = re.findall(r"\*\s*(\w+);", body)
    assert tuple(names) == SublayerBuffers.FIELDS
    assert re.findall(r"float (\w+);", body) == ["ln_eps"] and SublayerBuffers._fields_[-1][0] == "ln_eps"


@pytest.mark.parametrize("entry", ["metalllmSublayerEncode", "metalllmSublayerGraphCreate"])
def test_phase_encoder_validates_before_device(entry):
    """Both phases reject bad phases, shapes (the GEMM rules and the attention rules: M % 64,
    D in {64, 128}), NULL and misaligned buffers without touching the device."""
    from metalllm_amd.sublayer import SublayerBuffers, _L
    lib = _L()
    f = getattr(lib, entry)
    out = ctypes.c_void_p()
    last = ctypes.byref(out) if entry.endswith("Create") else None

    def call(phase, b, p):
        return f(phase, ctypes.byref(b) if b is not None else None, ctypes.byref(p) if p is not None else None, last)

    full = SublayerBuffers(*[(1 << 20) + 256 * i for i in range(len(SublayerBuffers.FIELDS))])
    good = dict(M=256, N=384, D=64, NH=6, B=1)
    P = lambda **c: AttentionParams(*[{**good, **c}[k] for k in ("M", "N", "D", "NH", "B")])
    for phase in (0, 1):
        assert call(phase, None, P()) == -1
        assert call(phase, full, None) == -1
        for change, code in ((dict(M=0), -2), (dict(M=96), -2), (dict(D=96, N=576), -3), (dict(D=32, N=192), -3),
                             (dict(N=383), -4), (dict(B=0), -4), (dict(B=1 << 12, M=1 << 16), -5)):
            assert call(phase, full, P(**change)) == code, (phase, change)
    assert call(2, full, P()) == -4
    assert call(-1, full, P()) == -4
    # a NULL or misaligned buffer the phase uses
    for name, phases in (("X", (0, 1)), ("out", (0,)), ("dOut", (1,)), ("dProjw", (1,)), ("l", (0, 1))):
        for phase in phases:
            b = SublayerBuffers(*[getattr(full, n) for n in SublayerBuffers.FIELDS])
            setattr(b, name, None)
            assert call(phase, b, P()) == -1, (name, phase)
            setattr(b, name, getattr(full, name) + 4)
            assert call(phase, b, P()) == -6, (name, phase)
    b = SublayerBuffers(*[getattr(full, n) for n in SublayerBuffers.FIELDS])
    b.dX_bf16 = full.dX_bf16 + 2  # optional, but aligned when given
    assert call(1, b, P()) == -6
    # the block fields: all or none once `hidden` is set; N <= 4096 for the layernorm; eps >= 0
    blk = ("ln_gamma", "ln_beta", "ln_xnorm", "ln_stdev", "ln_dgamma", "ln_dbeta", "residual", "dStream")
    for phase in (0, 1):
        b = SublayerBuffers(*[getattr(full, n) for n in SublayerBuffers.FIELDS], 1e-5)
        for name in blk:
            setattr(b, name, None)
        b.hidden = full.hidden
        assert call(phase, b, P()) == -1
        for name in blk:
            setattr(b, name, getattr(full, name))
        b.ln_eps = -1.0
        assert call(phase, b, P()) == -4
        b.ln_eps = 1e-5
        b.residual = full.residual + 8
        assert call(phase, b, P()) == -6
    if entry.endswith("Create"):
        assert lib.metalllmSublayerGraphCreate(0, ctypes.byref(full), ctypes.byref(P()), None) == -1
        assert out.value is None
        assert lib.metalllmSublayerGraphLaunch(None, None) == -1
        assert lib.metalllmSublayerGraphDestroy(None) == 0


def test_glue_entry_points_validate_before_device():
    """residualAdd and the layernorm kernels reject bad parameters, NULL and misaligned pointers
    without a device call."""
    from metalllm_amd.glue import LayernormParams, _L
    lib = _L()
    ok = ctypes.c_void_p(1 << 20)
    mis = ctypes.c_void_p((1 << 20) + 2)
    assert lib.residualAdd(None, None, None, 0, None) == 0
    assert lib.residualAdd(ok, None, ok, 8, None) == -1
    assert lib.residualAdd(ok, ok, mis, 8, None) == -6
    good = LayernormParams.of(64, 768)
    for bad, code in ((LayernormParams.of(0, 768), -4), (LayernormParams.of(64, 0), -4),
                      (LayernormParams.of(64, 100), -4), (LayernormParams.of(64, 4104), -4),
                      (LayernormParams(64, 768, 768, float("nan")), -4), (LayernormParams(64, 768, 768, -1.0), -4),
                      (LayernormParams.of(1 << 20, 4096), -5)):
        assert lib.layernormForward(ok, ok, ok, ok, ok, ok, ctypes.byref(bad), None) == code
        assert lib.layernormBackward(ok, ok, ok, ok, ok, ok, ok, ctypes.byref(bad), None) == code
    assert lib.layernormForward(ok, ok, ok, ok, ok, ok, None, None) == -1
    assert lib.layernormForward(ok, None, ok, ok, ok, ok, ctypes.byref(good), None) == -1
    assert lib.layernormForward(ok, ok, ok, mis, ok, ok, ctypes.byref(good), None) == -6
    assert lib.layernormBackward(ok, ok, ok, ok, ok, None, ok, ctypes.byref(good), None) == -1
    assert lib.layernormBackward(ok, ok, ok, ok, mis, ok, ok, ctypes.byref(good), None) == -6  # dx_norm, when given
    assert ctypes.sizeof(LayernormParams) == 16
