"""Benchmark of the causal attention hot path (flashAttentionForward + computeD +
flashAttentionBackward) on one MI355X, through the C ABI.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3] [--no-cpu-baseline]

One step = flashAttentionForward + computeD + the backward over one batch of synthetic bf16 inputs
already resident in HBM (the reference's per-layer sequence, model.h:459-473, 639-665). The
backward is flashAttentionBackwardWorkspace (dK/dV kernel storing dS into a device workspace, then
dQ = dS.K; workspace allocated once, outside the timed region, like the other buffers); the
recomputing flashAttentionBackward is timed beside it ("bwd_recompute"). Prints ONE JSON line.
FLOPs use the causal FlashAttention convention (half of dense): fwd 2*B*H*T^2*D, bwd
5*B*H*T^2*D, step 7*B*H*T^2*D.

The roofline object describes the dominant kernel, the dK/dV kernel (mla::bwd_kernel with the dS
store; the bench launches the backward's two kernels through metalllmAttnBackwardPart so that
each has its own events): its algorithmic FLOPs per launch (4 causal products: S, dP, dV, dK) over
its average launch time measured with HIP events on the launch stream, against MI355X dense bf16
matrix peak. roofline_dq does the same for the HBM-bound dQ kernel (bytes of dS, K and dQ per
launch against 8 TB/s). cpu_baseline times the CPU oracle (the scalar C++ transcription of the
reference math, oracle/attn_oracle.cpp) on a bounded sample of the same workload on this host's
cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 matrix peak
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    # id: (B, H, T, D, qk_scale, description)
    1: (128, 6, 256, 64, 1.0, "metalLLM training shape, larger batch"),
    2: (32, 12, 1024, 64, 1.5, "GPT-2-small-like, Q/K x1.5"),
    3: (16, 16, 4096, 128, 1.0, "long-context D=128 (target shape)"),
}


def flops(B, H, T, D):
    base = B * H * T * T * D
    return 2.0 * base, 5.0 * base


def traffic_from_profiles(cfg_id, kernel="bwd_dkdv"):
    """HBM bytes per launch of a kernel measured by rocprofv3 --pmc, if a summary was committed."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_traffic_config{cfg_id}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("bytes_per_launch")


def cpu_baseline(B, H, T, D, qk_scale, threads, target_s=10.0):
    """Times the oracle (fwd + computeD + bwd) with the plain sequential fp32 products of the
    reference's published matmul semantics (GEMM_SEQ) on whole batches (all heads), growing the
    sample until it takes about target_s; the oracle's bit-level matrix-core model (GEMM_MFMA,
    used by the parity tests) is timed once on batch 0 beside it."""
    import numpy as np
    import oracle as O

    def run(nb, heads, model):
        o = O.opts(threads=threads, gemm_model=model)
        q = O.normal_bf16((nb, T, heads, D), 1, O.TID_Q, qk_scale)
        k = O.normal_bf16((nb, T, heads, D), 1, O.TID_K, qk_scale)
        v = O.normal_bf16((nb, T, heads, D), 1, O.TID_V)
        g = O.normal_bf16((nb, T, heads, D), 1, O.TID_DO)
        t0 = time.perf_counter()
        out, lse = O.forward(q, k, v, o)
        Dv = O.compute_d(g, out, o)
        O.backward(g, Dv, lse, q, k, v, o)
        dt = time.perf_counter() - t0
        ff, fb = flops(nb, heads, T, D)
        return (ff + fb) / dt / 1e12, dt

    nb = 1
    rate, dt = run(nb, H, O.GEMM_SEQ)
    if dt < target_s / 2 and B > 1:
        nb = int(min(B, max(2, round(nb * target_s / max(dt, 1e-3)))))
        rate, dt = run(nb, H, O.GEMM_SEQ)
    heads_m = min(H, threads)
    rate_m, dt_m = run(1, heads_m, O.GEMM_MFMA)
    return {
        "value": rate,
        "unit": "TFLOP/s",
        "cores": threads,
        "host_cores": len(os.sched_getaffinity(0)),
        "kind": "port",
        "sample": f"b=0..{nb - 1}, all {H} heads (T={T}, D={D}): fwd+computeD+bwd of the oracle (scalar C++ "
                  f"transcription, plain sequential fp32 products), {dt:.1f} s on {threads} threads; the rate "
                  f"scales to the full batch",
        "mfma_model": {"value": rate_m, "seconds": round(dt_m, 1),
                       "sample": f"b=0, {heads_m} heads, the oracle's bit-level matrix-core product model"},
    }


def bench_sublayer(args, shape=(8, 2048, 768, 12), label="config4"):
    """one pre-LN block's attention sublayer, fwd + bwd, X bf16 [8, 2048, 768]
    ~N(0,1), Wq/Wk/Wv/Wproj bf16 [768, 768] ~N(0, 0.02), dOut ~N(0,1), H=12 (D=64). One step =
    forward computeQKV -> flashAttentionForward -> projForward and backward projBackwarddW/dX ->
    computeD -> flashAttentionBackward -> computeGradDx/Dw (model.h:446-482, 621-690), with the
    accumulated gradients starting from zero (model.h:549-555). The per-call chain (timed per phase
    by events) zeroes them and adds into them; the headline, the phase encoder, writes them as
    0 + the gradient. Returns the result object (ms per step and the attention share).
    `shape` = (B, T, C, H) runs the same chain at another shape; (128, 256, 384, 6) is config 1's
    attention shape (metalLLM's own N_EMBED = 384, 6 heads), where the step is short enough for the
    host's launch cost to show between the per-call chain, the encoder and the graphs."""
    import torch
    import metalllm_amd as M
    from metalllm_amd import sublayer as S
    B, T, C, H = shape
    D = C // H
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(4321)
    rn = lambda shape, sc=1.0: (torch.randn(shape, generator=gen, device=dev) * sc).to(torch.bfloat16)
    X = rn((B, T, C))
    # q_w, k_w, v_w as slices of one fused [3, C, C] weight (computeQKV then runs one batched product)
    Ws = list(rn((3, C, C), 0.02).unbind(0)) + [rn((C, C), 0.02)]
    dOut = rn((B, T, C))
    sub = S.Sublayer(X, *Ws, H=H)
    stream = torch.cuda.current_stream()
    names = ["zero", "qkv", "attn_fwd", "proj_fwd", "proj_bwd", "attn_bwd", "grad_dx_dw"]

    def step(ev=None):
        rec = (lambda i: ev[i].record(stream)) if ev is not None else (lambda i: None)
        rec(0)
        sub.zero_grads()
        rec(1)
        S.computeQKV(sub.X, sub.q, sub.k, sub.v, sub.Wq, sub.Wk, sub.Wv, sub.p, stream)
        rec(2)
        M.flashAttentionForward(sub.q, sub.k, sub.v, sub.o, sub.lse, stream, sub.p)
        rec(3)
        S.projForward(sub.o, sub.Wp, sub.out, sub.p, stream)
        rec(4)
        marks = {"proj": 5, "attention": 6, "grads": 7}
        sub.backward(dOut, stream, parts=lambda name: rec(marks[name]))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(8)] for _ in range(args.steps)]
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(events[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_calls = wall * 1e3 / args.steps
    phase = {n: sorted(e[i].elapsed_time(e[i + 1]) for e in events)[args.steps // 2] for i, n in enumerate(names)}
    attn = phase["attn_fwd"] + phase["attn_bwd"]
    total_events = sum(phase.values())
    gemm_flop = 12 * 2.0 * B * T * C * C
    attn_flop = 7.0 * B * H * T * T * D

    # The same step through the phase encoder: both phases enqueued by the library
    # (metalllmSublayerEncode), then recorded once as HIP graphs and replayed. The same products
    # and the same results: phase 1 writes dX and the weight gradients as 0 + the gradient (bit
    # for bit what the per-call chain's zeroing and accumulation give) instead of zeroing them
    # and adding into them, and reads dOut from the sublayer's buffer; the dX cast of model.h:692
    # is left out (it is not part of config 4's chain).
    sub.dOut.copy_(dOut)

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t) * 1e3 / args.steps

    bufs = sub.buffers(cast=False)
    ms_encode = timed(lambda: (S.encode_phase(0, bufs, sub.p, stream), S.encode_phase(1, bufs, sub.p, stream)))
    graphs = (S.PhaseGraph(0, bufs, sub.p), S.PhaseGraph(1, bufs, sub.p))
    ms_graph = timed(lambda: (graphs[0].launch(stream), graphs[1].launch(stream)))
    for g in graphs:
        g.close()
    if args.calibrate_copy:
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
    ms = ms_encode
    sub.close()
    return {
        "metric": f"attention sublayer fwd+bwd ms per step ({label}), with the attention share",
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{label}: pre-LN attention sublayer fwd+bwd (QKV, causal flash attention, "
                               "projection; their gradients)", "B": B, "T": T, "C": C, "H": H, "D": D},
        "step_mode": "phase encoder (metalllmSublayerEncode, one call per phase)",
        "modes_ms_per_step": {"graph": round(ms_graph, 4), "encoder": round(ms_encode, 4),
                              "per_call": round(ms_calls, 4)},
        "attention_share": round(attn / ms, 4),
        "phases_ms_median": {k: round(v, 4) for k, v in phase.items()},
        "tflops": {"step": round((gemm_flop + attn_flop) / (ms * 1e-3) / 1e12, 2),
                   "gemms": round(gemm_flop / ((total_events - attn - phase["zero"]) * 1e-3) / 1e12, 2),
                   "attention": round(attn_flop / (attn * 1e-3) / 1e12, 2)},
    }


def step_bound_ms(B, H, T, D):
    """Roofline time of one attention step (fwd + computeD + bwd): per kernel the larger of its
    algorithmic bytes at 8 TB/s and its causal FLOPs at the dense bf16 peak, summed."""
    bthd, bht = B * T * H * D, B * H * T
    ff, fb = flops(B, H, T, D)
    fwd = max((8 * bthd + 4 * bht) / PEAK_HBM_GBS / 1e9, ff / PEAK_BF16_TFLOPS / 1e12)
    cd = (4 * bthd + 4 * bht) / PEAK_HBM_GBS / 1e9
    bwd = max((16 * bthd + 8 * bht) / PEAK_HBM_GBS / 1e9, fb / PEAK_BF16_TFLOPS / 1e12)
    return 1e3 * (fwd + cd + bwd), 1e3 * fwd, 1e3 * bwd


def run_core(cfg_id, steps, warmup, calibrate_copy=False):
    """Times the attention core of one config (fwd + computeD + backward, inputs resident in HBM).
    Two step kinds: the headline step with flashAttentionBackwardWorkspace (parts 2 and 3) and the
    reference-contract step with flashAttentionBackward (parts 0 and 1, into a zeroed dQ, the
    memset included). Returns the per-kernel event spans and both steps' spans."""
    import torch
    import metalllm_amd as M

    B, H, T, D, qk_scale, desc = CONFIGS[cfg_id]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    shape = (B, T, H, D)

    def randn(scale=1.0):
        return (torch.randn(shape, generator=gen, device=dev, dtype=torch.float32) * scale).to(torch.bfloat16)

    q, k, v, dO = randn(qk_scale), randn(qk_scale), randn(), randn()
    # written between timed steps (outside the events) so that no input is served from the 256 MB
    # Infinity Cache or the L2s of the previous step
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    out = torch.empty_like(q)
    lse = torch.empty((B, H, T), dtype=torch.float32, device=dev)
    Dv = torch.empty_like(lse)
    dQ = torch.empty(shape, dtype=torch.float32, device=dev)
    dK = torch.empty_like(q)
    dV = torch.empty_like(q)
    ws_bytes = M.workspace_bytes(B, T, H, D)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    p = M.AttentionParams.of(B, T, H, D)

    # flashAttentionBackwardWorkspace == part 2 (dK/dV kernel + dS store) then part 3 (dQ from dS);
    # flashAttentionBackward == part 0 then part 1. The bench launches the parts itself so that
    # each kernel is timed by its own events. The workspace path writes dQ in full; the
    # recomputing path adds into dQ (the reference's contract), so its steps zero dQ first.
    # ev: None (untimed), 5 events (a marker before, between and after the kernels: the phase
    # spans) or 2 events (start and end only: the step span, free of the markers' own cost,
    # which is a few microseconds each)
    def step(ev=None, parts=(2, 3)):
        flush.fill_(parts[0])
        mark = (lambda i: ev[i].record(stream)) if ev is not None and len(ev) == 5 else (lambda i: None)
        if ev is not None:
            ev[0].record(stream)
        M.flashAttentionForward(q, k, v, out, lse, stream, p)
        mark(1)
        M.computeD(dO, out, Dv, stream, p)
        mark(2)
        if parts[0] == 0:
            dQ.zero_()  # the memset the reference's caller does (model.h:549), timed with the backward
        M.backward_part(parts[0], dO, Dv, lse, q, k, v, dQ, dK, dV, stream, p, workspace=ws)
        mark(3)
        M.backward_part(parts[1], dO, Dv, lse, q, k, v, dQ, dK, dV, stream, p, workspace=ws)
        if ev is not None:
            ev[-1].record(stream)

    def timed_steps(parts, n, nev):
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(nev)] for _ in range(n)]
        for e in evs:
            step(e, parts=parts)
        torch.cuda.synchronize()
        return evs

    # the reference-contract step (flashAttentionBackward): its own warmup, phase and step spans
    n_rc = max(3, steps // 4)
    for _ in range(2):
        step(parts=(0, 1))
    rc_events = timed_steps((0, 1), n_rc, 5)
    rc_plain = timed_steps((0, 1), n_rc, 2)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # phase spans: steps with markers between the kernels
    events = timed_steps((2, 3), steps, 5)
    # headline: the same steps with one event pair each
    t0 = time.perf_counter()
    plain = timed_steps((2, 3), steps, 2)
    wall = time.perf_counter() - t0

    if calibrate_copy:
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()

    span = lambda a, b, evs=events: sorted(e[a].elapsed_time(e[b]) for e in evs)
    res = {
        "shape": (B, H, T, D, qk_scale, desc), "ws_bytes": ws_bytes,
        "fwd": span(0, 1), "cd": span(1, 2), "kv": span(2, 3), "dq": span(3, 4), "bwd": span(2, 4),
        "marked": span(0, 4), "step": span(0, 1, plain), "wall_ms": wall * 1e3 / steps,
        "rc_kv": span(2, 3, rc_events), "rc_dq": span(3, 4, rc_events), "rc_bwd": span(2, 4, rc_events),
        "rc_step": span(0, 1, rc_plain),
    }
    del q, k, v, dO, flush, out, lse, Dv, dQ, dK, dV, ws
    torch.cuda.empty_cache()
    return res


def med(xs):
    return xs[len(xs) // 2]


def core_summary(cfg_id, r):
    """Compact per-config record (the extra configs of the default run)."""
    B, H, T, D, qk_scale, desc = r["shape"]
    ff, fb = flops(B, H, T, D)
    bound, bound_f, bound_b = step_bound_ms(B, H, T, D)
    ms, rc_ms = med(r["step"]), med(r["rc_step"])
    regime = "hbm" if cfg_id == 1 else ("ridge" if cfg_id == 2 else "mfma")
    return {
        "workload": f"config{cfg_id}: causal attention fwd+computeD+bwd, {desc}",
        "B": B, "H": H, "T": T, "D": D, "qk_scale": qk_scale,
        "ms_per_step": round(ms, 4),
        "tflops": round((ff + fb) / (ms * 1e-3) / 1e12, 2),
        "pct_of_peak": round(100.0 * (ff + fb) / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
        "bound": {"regime": regime, "step_ms": round(bound, 4), "fwd_ms": round(bound_f, 4),
                  "bwd_ms": round(bound_b, 4),
                  "note": "per kernel max(algorithmic bytes / 8 TB/s, causal FLOPs / 2516.6 TFLOP/s), summed "
                          "over fwd, computeD and bwd"},
        "frac_of_bound": round(bound / ms, 4),
        "phases_ms_median": {"fwd": round(med(r["fwd"]), 4), "computeD": round(med(r["cd"]), 4),
                             "bwd": round(med(r["bwd"]), 4), "bwd_dkdv": round(med(r["kv"]), 4),
                             "bwd_dq": round(med(r["dq"]), 4)},
        "ref_contract_step": {"ms_per_step": round(rc_ms, 4),
                              "tflops": round((ff + fb) / (rc_ms * 1e-3) / 1e12, 2),
                              "bwd_ms_median": round(med(r["rc_bwd"]), 4)},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3, choices=sorted(CONFIGS) + [4],
                    help="1-3: attention core (fwd + computeD + bwd); 4: the whole attention sublayer")
    ap.add_argument("--sublayer-shape", default=None, metavar="B,T,C,H",
                    help="with --config 4: run the sublayer chain at this shape instead of config 4's "
                         "(e.g. 128,256,384,6, config 1's attention shape)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="skip the other BASELINE configs that the default run measures beside the headline")
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="after the timed steps, run one device copy of 256 MiB (read) -> 256 MiB (write), "
                         "the known-size reference for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the single-GPU hot path only: attention shards per (batch, head) with no "
              "exchange, so this build runs and reports one GPU (use --gpus 1).", file=sys.stderr)
        sys.exit(2)

    import torch  # noqa: F401
    import metalllm_amd as M  # noqa: F401

    if args.config == 4:
        if args.sublayer_shape:
            shape = tuple(int(x) for x in args.sublayer_shape.split(","))
            if len(shape) != 4 or min(shape) < 1 or shape[2] % shape[3]:
                ap.error("--sublayer-shape takes B,T,C,H: positive, with H dividing C")
            r = bench_sublayer(args, shape=shape, label="config4 chain at B,T,C,H = " + args.sublayer_shape)
        else:
            r = bench_sublayer(args)
        print(json.dumps(r), flush=True)
        return
    r = run_core(args.config, args.steps, args.warmup, args.calibrate_copy)
    B, H, T, D, qk_scale, desc = r["shape"]
    ws_bytes = r["ws_bytes"]
    fwd_ms, cd_ms, kv_ms, dq_ms, bwd_ms = r["fwd"], r["cd"], r["kv"], r["dq"], r["bwd"]
    avg = lambda xs: sum(xs) / len(xs)
    ff, fb = flops(B, H, T, D)
    unit = B * H * T * T * D  # one causal T x T x D product over all (b, h)
    # headline: the median over the timed steps of each step's event span (one pair around the
    # kernels); the wall-clock mean of those steps (which also covers the cache flush between
    # steps) is reported beside it, and so is the span of the marked steps
    ms_per_step = med(r["step"])
    marked_ms = med(r["marked"])
    value = (ff + fb) / (ms_per_step * 1e-3) / 1e12
    # dominant kernel: the dK/dV kernel (4 products: S, dP, dV = P^T dO, dK = dS^T Q)
    kv_avg = avg(kv_ms)
    achieved = 4.0 * unit / (kv_avg * 1e-3) / 1e12
    # dQ kernel from the stored dS: reads every dS tile once, K (once per 128-query block, from L2
    # after the first), writes dQ fp32 once; algorithmic bytes = dS + K + dQ
    bthd = B * T * H * D
    dq_bytes = ws_bytes + 2 * bthd + 4 * bthd
    dq_avg = avg(dq_ms)
    rc_kv, rc_dq, rc_bwd = r["rc_kv"], r["rc_dq"], r["rc_bwd"]

    if D == 64 and T <= 256:
        # short sequences: one fused kernel (part 2) computes dK, dV and dQ without the workspace
        # (part 3 launches nothing); at T = 256 the backward is HBM-bound (5T/16 FLOP per byte)
        bwd_bytes = 16 * bthd + 8 * B * H * T
        roofline = {
            "kernel": "fused short-sequence backward (mla::bwd_short_kernel<false>: dK, dV and dQ)",
            "bound": "hbm",
            "achieved": round(bwd_bytes / (kv_avg * 1e-3) / 1e9, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(bwd_bytes / (kv_avg * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "traffic": traffic_from_profiles(args.config, "bwd_short"),
            "algorithmic_bytes": bwd_bytes,
            "tflops": round(5.0 * unit / (kv_avg * 1e-3) / 1e12, 2),
            "avg_ms": round(kv_avg, 4),
        }
        roofline_dq = None
    elif D == 64:
        # the workspace entry point runs the recomputing kernels at D = 64 (no dS stored): dK/dV
        # (4 products: S, dP, dV, dK) and dQ written (3 products: S, dP, dQ)
        roofline = {
            "kernel": "backward dK/dV kernel without the dS store (mla::bwd_kernel<64, false>; at D = 64 "
                      "the workspace entry point recomputes dS instead of storing it)",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": None,
            "algorithmic_bytes": 12 * bthd + 8 * B * H * T,
            "avg_ms": round(kv_avg, 4),
        }
        dq_exec = 3.0 * unit / (dq_avg * 1e-3) / 1e12
        roofline_dq = {
            "kernel": "backward dQ kernel recomputing S, dP and dS, dQ written (mla::bwd_dq_kernel<64, false>)",
            "bound": "mfma",
            "achieved": round(dq_exec, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(dq_exec / PEAK_BF16_TFLOPS, 4),
            "traffic": None,
            "note": "three executed products per launch (S, dP, dQ); one of them (dQ) is algorithmic",
            "avg_ms": round(dq_avg, 4),
        }
    else:
        roofline = {
            "kernel": "backward dK/dV kernel with the dS store (mla::bwd_kernel<D, true>)",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic_from_profiles(args.config),
            # the kernel's share of the backward's algorithmic bytes (Q, K, V, dO read; dK, dV
            # written; lse, D read); the dS tiles it stores for the dQ kernel are design traffic
            "algorithmic_bytes": 12 * bthd + 8 * B * H * T,
            "workspace_write_bytes": ws_bytes,
            "avg_ms": round(kv_avg, 4),
        }
        roofline_dq = {
            "kernel": "backward dQ kernel from the stored dS (mla::dqs_kernel)",
            "bound": "hbm",
            "achieved": round(dq_bytes / (dq_avg * 1e-3) / 1e9, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(dq_bytes / (dq_avg * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "traffic": traffic_from_profiles(args.config, "dqs"),
            "algorithmic_bytes": dq_bytes,
            "note": "bytes this kernel must move (stored dS + K + dQ); the backward's algorithmic bytes "
                    "(16*BTHD + 8*BHT) do not include the dS round trip",
            "avg_ms": round(dq_avg, 4),
        }

    rc_ms = med(r["rc_step"])
    result = {
        "metric": "causal attn fwd+bwd TFLOP/s at B,H,T,D bf16; % of MI355X bf16 MFMA peak",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"config{args.config}: causal attention fwd+computeD+bwd, {desc}",
                   "B": B, "H": H, "T": T, "D": D, "qk_scale": qk_scale, "causal": True},
        "pct_of_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "timing": "median of per-step HIP event spans (one event pair around fwd, computeD and bwd); "
                  "512 MB written between steps (L2 and Infinity Cache flush); phases from as many steps "
                  "again with a marker between the kernels",
        "wall_ms_per_step_incl_flush": round(r["wall_ms"], 4),
        "marked_ms_per_step": round(marked_ms, 4),
        "phases": {
            "fwd_ms_median": round(med(fwd_ms), 4), "computeD_ms_median": round(med(cd_ms), 4),
            "bwd_ms_median": round(med(bwd_ms), 4), "bwd_dkdv_ms_median": round(med(kv_ms), 4),
            "bwd_dq_ms_median": round(med(dq_ms), 4),
            "bwd_recompute_ms_median": round(med(rc_bwd), 4), "bwd_recompute_dkdv_ms_median": round(med(rc_kv), 4),
            "bwd_recompute_dq_ms_median": round(med(rc_dq), 4),
            "workspace_bytes": ws_bytes,
            "fwd_tflops": round(ff / (med(fwd_ms) * 1e-3) / 1e12, 2),
            "bwd_tflops": round(fb / (med(bwd_ms) * 1e-3) / 1e12, 2),
            "computeD_gbs": round((4 * bthd + 4 * B * H * T) / (med(cd_ms) * 1e-3) / 1e9, 1),
        },
        # the step the reference's own entry point gives (model.h:648-665): flashAttentionBackward
        # (no workspace, dQ accumulated into a zeroed buffer, the memset timed with it)
        "ref_contract_step": {
            "ms_per_step": round(rc_ms, 4),
            "tflops": round((ff + fb) / (rc_ms * 1e-3) / 1e12, 2),
            "pct_of_peak": round(100.0 * (ff + fb) / (rc_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
            "bwd_ms_median": round(med(rc_bwd), 4),
        },
        "roofline": roofline,
    }
    if roofline_dq is not None:
        result["roofline_dq"] = roofline_dq
    if not args.no_extra_configs:
        # the other BASELINE configs, measured in the same run (the headline stays config 3)
        extra = {}
        for cid in sorted(CONFIGS):
            if cid != args.config:
                extra[f"config{cid}"] = core_summary(cid, run_core(cid, args.steps, args.warmup))
        c4 = bench_sublayer(args)
        keys = ("config", "ms_per_step", "step_mode", "modes_ms_per_step", "attention_share",
                "phases_ms_median", "tflops")
        extra["config4"] = {k: c4[k] for k in keys}
        # the same sublayer at config 1's shape: the short step where launch cost can show
        c4s = bench_sublayer(args, shape=(128, 256, 384, 6), label="config4 chain at config 1's shape")
        extra["config4_at_config1_shape"] = {k: c4s[k] for k in keys}
        result["extra_configs"] = extra
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(B, H, T, D, qk_scale, args.cpu_threads)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
