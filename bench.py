#!/usr/bin/env python3
"""Benchmark of the MI355X projection path (one GPU).

Headline workload (decode M=1): one decode step of
the fused MLP block -- RMSNorm(1+w) prologue, gate/up GEMV with SiLU*mul,
down GEMV with residual add -- for all 24 layers of Qwen3.5-0.8B, BF16
weights N(0,0.02) random-initialised per layer, BF16 activations, FP32
accumulate.  24 distinct layers (528 MB of weights) exceed the 256 MB
Infinity Cache, so every step streams the weights from HBM.  The step is
one qw_mlp_stack call (all 24 blocks in one persistent launch that streams
block l+1's weights during block l's hand-offs), captured once in a HIP
graph and replayed; the same 24 blocks as 24 qw_mlp_fused launches are
reported under extra.

value = algorithmic bytes of the step / step time (GB/s), with
  per layer: W 22,020,096 B + x M*1024*2 + y M*1024*2 + gamma 1024*4.
roofline: the dominant kernel -- the persistent MLP stack kernel
(qwk::mlp_stack_kernel, 528.5 MB of weights per launch), which is the whole
headline step (one launch) -- timed with HIP events on the step's own stream
over the timed region.
cpu_baseline: the reference's own MLP::forward_batch (oracle/_ref, compiled
from the reference sources; FP32, 1 thread) on a bounded sample, expressed
in the same algorithmic-bytes unit.  Falls back to the oracle port when
oracle/_ref is absent.

Sub-measurements for the other BASELINE configs are reported under "extra".
"""
import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "qwen3.5_0.8b_deploy_amd")
HBM_PEAK = 8000.0        # GB/s, MI355X
BF16_PEAK = 2500.0       # TFLOP/s dense
H, I, V = 1024, 3584, 248320
LAYERS = 24
LINEAR_LAYERS = [i for i in range(24) if i % 4 != 3]   # 18 Gated-DeltaNet layers
COPY_BYTES = 64 << 20   # calibration copy for the HBM traffic counters
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_mlp_stack_bf16_M1.txt")
METRIC = "decode GEMV HBM GB/s (% of peak) at M=1; prefill GEMM TFLOPS (% MFMA peak)"


def load_qw():
    spec = importlib.util.spec_from_file_location("qw", os.path.join(PKG, "qw.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timer:
    """HIP-event timing of a callable replayed `steps` times on `stream`."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream

    def run(self, fn, steps, warmup):
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record(self.stream)
            for _ in range(steps):
                fn()
            t1.record(self.stream)
            torch.cuda.synchronize()
        return t0.elapsed_time(t1) / steps   # ms per step


def graphed(qw, ctx, stream, body):
    """Capture body() into a HIP graph (through the library's graph API)."""
    import torch
    with torch.cuda.stream(stream):
        body()                               # one eager pass first
        torch.cuda.synchronize()
        g = qw.Graph(ctx, stream)
        with g:
            body()
    return g


def mlp_bytes(M):
    return 3 * H * I * 2 + M * H * 2 * 2 + H * 4


def gateup_bytes(M):
    return 2 * H * I * 2 + M * H * 2 + M * I * 2 + H * 4


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE counter runs, each scaled by what the
    same counter reads for a 64 MiB copy; None when the summary is absent."""
    try:
        vals = {}
        with open(TRAFFIC_FILE) as f:
            for line in f:
                k, sep, v = line.partition(":")
                if sep and k.strip() in ("copy_bytes", "copy_fetch_kib", "copy_write_kib",
                                         "kernel_fetch_kib", "kernel_write_kib"):
                    vals[k.strip()] = float(v)
        ff = vals["copy_bytes"] / (vals["copy_fetch_kib"] * 1024)
        fw = vals["copy_bytes"] / (vals["copy_write_kib"] * 1024)
        return int(vals["kernel_fetch_kib"] * 1024 * ff + vals["kernel_write_kib"] * 1024 * fw)
    except (OSError, KeyError, ValueError, ZeroDivisionError):
        return None


def cpu_baseline(oracle):
    """Reference CPU MLP (1 thread) on a bounded sample of the same workload."""
    ref = oracle.ref_lib()
    Wg = oracle.normal((I, H), 1, 0.0, 0.02)
    Wu = oracle.normal((I, H), 2, 0.0, 0.02)
    Wd = oracle.normal((H, I), 3, 0.0, 0.02)
    x = oracle.normal((1, H), 4)
    y = np.empty((1, H), np.float32)
    if ref is not None:
        t1 = ref.ref_mlp_time(Wg, Wu, Wd, x, y, 1, H, I, 1)
        iters = max(1, min(10000, int(12.0 / max(t1, 1e-4))))
        secs = ref.ref_mlp_time(Wg, Wu, Wd, x, y, 1, H, I, iters)
        kind = "reference"
        what = "qwen::MLP::forward_batch (reference language_mlp.cpp, built -O2 by oracle/Makefile)"
    else:
        t0 = time.perf_counter(); oracle.mlp(Wg, Wu, Wd, x); t1 = time.perf_counter() - t0
        iters = max(1, min(10000, int(12.0 / max(t1, 1e-4))))
        t0 = time.perf_counter()
        for _ in range(iters):
            oracle.mlp(Wg, Wu, Wd, x)
        secs = time.perf_counter() - t0
        kind = "port"
        what = "orc_mlp (oracle restatement of language_mlp.cpp:53-91)"
    per = secs / iters
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(mlp_bytes(1) / per / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": kind,
        "sample": (f"{iters} MLP blocks at M=1 (H=1024, I=3584, FP32 weights) in {secs:.1f} s "
                   f"= {per * 1e3:.2f} ms/block via {what}; RMSNorm+residual not included; "
                   f"host {cpu_model!r}, nproc={os.cpu_count()}"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline only (no extra configs)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="", help="comma-separated extra workloads to run (cfg1, cfg2, cfg3, wide, "
                    "int8gemv, prefill, gdn, attn, model, lmhead; decode1 = the B=1 decode step of model alone; default all), e.g. for a profiler pass over one of them")
    ap.add_argument("--profile-kernel", action="store_true",
                    help="counter pass: only the dominant kernel (4 eager MLP stack launches) and a "
                         "64 MiB calibration copy, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(requested --gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    qw = load_qw()
    torch.cuda.set_device(0)
    # workspace sized for the M=16384 prefill stack (RMSNorm-ed activations)
    ctx = qw.Context(0, qw.lib().qw_workspace_query(16384, 8224, 4096))
    stream = torch.cuda.Stream()
    timer = Timer(torch, stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)

    def randn(*shape, std=1.0, dtype=torch.bfloat16):
        return (torch.randn(*shape, generator=gen, device="cuda") * std).to(dtype)

    # ---------------- headline: 24-layer fused MLP decode step, BF16, M=1 ----
    log("building 24 BF16 MLP layers ...")
    gu, dn, gam = [], [], []
    for _ in range(LAYERS):
        g, u = randn(I, H, std=0.02), randn(I, H, std=0.02)
        gu.append(qw.Weight.pack_glu_device(ctx, g, u, qw.WFMT_BF16))
        d = randn(H, I, std=0.02)
        dn.append(qw.Weight.pack_device(ctx, d, qw.WFMT_BF16))
        gam.append(randn(H, std=0.02, dtype=torch.float32))
        del g, u, d
    torch.cuda.synchronize()

    def mlp_step(hbuf, M):
        def body():
            for l in range(LAYERS):
                qw.mlp_fused(ctx, gu[l], dn[l], hbuf, hbuf, gamma=gam[l], residual=hbuf)
        return body

    h1 = randn(1, H)
    if args.profile_kernel:
        with torch.cuda.stream(stream):
            for _ in range(4):
                qw.mlp_stack(ctx, gu, dn, h1, h1, gammas=gam, stream=stream)
            src = torch.empty(COPY_BYTES // 2, device="cuda", dtype=torch.bfloat16).fill_(1.0)
            dst = torch.empty_like(src)
            for _ in range(4):
                dst.copy_(src)
        torch.cuda.synchronize()
        log("profile pass done")
        ctx.close()
        return
    g_mlp = graphed(qw, ctx, stream, lambda: qw.mlp_stack(ctx, gu, dn, h1, h1, gammas=gam, stream=stream))
    ms = timer.run(g_mlp.launch, args.steps, args.warmup)
    step_bytes = LAYERS * mlp_bytes(1)
    value = step_bytes / (ms * 1e-3) / 1e9
    err = ctx.device_error()
    if err:
        raise RuntimeError(f"device error flag {err} after the headline step")
    log(f"headline: {ms * 1e3:.1f} us/step, {value:.0f} GB/s")

    # Dominant kernel: the persistent MLP stack kernel, one launch per step.
    # Its average launch duration is the timed region of the step graph (HIP
    # events on the stream the kernel runs on) over the launches, so it
    # includes the graph's launch gap and is an upper bound.
    k_us = ms * 1e3
    k_bytes = step_bytes
    k_gbs = k_bytes / (k_us * 1e-6) / 1e9
    log(f"mlp stack kernel: {k_us:.2f} us avg, {k_gbs:.0f} GB/s")
    # the same 24 blocks as 24 one-launch MLP kernels (qw_mlp_fused)
    g_pl = graphed(qw, ctx, stream, mlp_step(h1, 1))
    pl_ms = timer.run(g_pl.launch, args.steps, args.warmup)
    log(f"per-block launches: {pl_ms * 1e3:.1f} us/step, {step_bytes / (pl_ms * 1e-3) / 1e9:.0f} GB/s")
    # the separate fused RMSNorm + gate/up + SiLU*mul GEMV (the two-launch form)
    hmid = torch.empty(1, I, device="cuda", dtype=torch.bfloat16)
    g_gu = graphed(qw, ctx, stream, lambda: [qw.linear(ctx, gu[l], h1, hmid, gamma=gam[l]) for l in range(LAYERS)])
    gu_us = 1e3 * timer.run(g_gu.launch, args.steps, args.warmup) / LAYERS
    log(f"gate/up kernel: {gu_us:.2f} us avg, {gateup_bytes(1) / (gu_us * 1e-6) / 1e9:.0f} GB/s")

    extra = {}
    if not args.quick:
        extra = run_extras(qw, ctx, torch, timer, stream, randn, gu, dn, gam, args)
    extra["gateup_glu_kernel_bf16_M1"] = {"us_per_launch": round(gu_us, 3),
                                          "GBps": round(gateup_bytes(1) / (gu_us * 1e-6) / 1e9, 1)}
    extra["mlp_per_block_launches_bf16_M1"] = {
        "us_per_step": round(pl_ms * 1e3, 1), "us_per_block": round(pl_ms * 1e3 / LAYERS, 2),
        "GBps": round(step_bytes / (pl_ms * 1e-3) / 1e9, 1),
        "pct_hbm": round(100 * step_bytes / (pl_ms * 1e-3) / 1e9 / HBM_PEAK, 1)}

    cpu = None
    if not args.no_cpu:
        import oracle
        log("cpu baseline ...")
        cpu = cpu_baseline(oracle)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) activations; random init, no checkpoint)",
        "config": {
            "workload": "fused MLP block decode step (RMSNorm+gate/up+SiLU*mul+down+residual), "
                        "24 Qwen3.5-0.8B layers, BF16 weights, M=1 (BASELINE configs[1]); one qw_mlp_stack "
                        "launch, HIP graph replay",
            "global_batch": 1, "seq_len": 1, "hidden": H, "intermediate": I, "layers": LAYERS,
            "bytes_per_step": step_bytes, "pct_of_hbm_peak": round(100 * value / HBM_PEAK, 2),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "qwk::mlp_stack_kernel<BF16 weights, BF16 x, gamma, M=1> (24 RMSNorm+gate/up+SiLU*mul+down+residual blocks, one persistent launch)",
            "achieved": round(k_gbs, 2),
            "peak": HBM_PEAK,
            "unit": "GB/s",
            "frac": round(k_gbs / HBM_PEAK, 4),
            "traffic": measured_traffic(),
            "algorithmic_bytes_per_launch": k_bytes,
            "avg_launch_us": round(k_us, 3),
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


def run_extras(qw, ctx, torch, timer, stream, randn, gu, dn, gam, args):
    extra = {}
    steps = max(5, args.steps // 2)
    only = set(filter(None, args.only.split(",")))
    want = lambda name: not only or name in only

    # config 2: fused MLP at decode batches.  The RMSNorm weight is a model
    # constant, so it is folded into the gate/up columns once at load time
    # (qw_weight_fold_norm); the kernels still normalize every token.
    gu_f = []
    if want("cfg2"):
        for l in range(LAYERS):
            g_, u_ = randn(I, H, std=0.02), randn(I, H, std=0.02)
            w = qw.Weight.pack_glu_device(ctx, g_, u_, qw.WFMT_BF16)
            w.fold_norm(gam[l])
            gu_f.append(w)
            del g_, u_
    # qw_mlp_stack: one persistent launch for all 24 blocks up to 8 tokens,
    # the 24 qw_mlp_fused launches beyond
    for M in ((8, 32, 128) if want("cfg2") else ()):
        hb = randn(M, H)
        g = graphed(qw, ctx, stream, lambda hb=hb: qw.mlp_stack(ctx, gu_f, dn, hb, hb, stream=stream))
        ms = timer.run(g.launch, steps, 2)
        b = LAYERS * mlp_bytes(M)
        fl = LAYERS * 2.0 * M * 3 * H * I
        extra[f"cfg2_mlp_bf16_M{M}"] = {"us_per_layer": round(ms * 1e3 / LAYERS, 2), "norm": "gamma folded into gate/up",
                                        "path": "persistent stack" if M <= 8 else "per-block launches",
                                        "GBps": round(b / ms / 1e6, 1),
                                        "TFLOPs": round(fl / ms / 1e9, 2),
                                        "tok_per_s_stack": round(M / (ms * 1e-3), 1)}
        log("cfg2", M, extra[f"cfg2_mlp_bf16_M{M}"])

    extra.update(run_cfg1(qw, ctx, torch, timer, stream, randn, steps) if want("cfg1") else {})
    extra.update(run_cfg3(qw, ctx, torch, timer, stream, randn, steps) if want("cfg3") else {})
    del gu_f
    extra.update(run_int8_gemv(qw, ctx, torch, timer, stream, randn, steps) if want("int8gemv") else {})
    extra.update(run_wide(qw, ctx, torch, timer, stream, randn, steps) if want("wide") else {})
    if want("prefill"):
        extra.update(run_prefill(qw, ctx, torch, timer, stream, randn, args))
    if want("gdn"):
        extra.update(run_gdn(qw, ctx, torch, timer, stream, randn, args))
    if want("attn"):
        extra.update(run_attn(qw, ctx, torch, timer, stream, randn, args))
    if want("model") or (only and "decode1" in only):
        extra.update(run_decode_model(qw, ctx, torch, timer, stream, randn, args, b1_only=not want("model")))
    if want("lmhead"):
        extra.update(run_lmhead(qw, ctx, torch, timer, stream, randn, steps))
    torch.cuda.synchronize()
    return extra


def run_cfg1(qw, ctx, torch, timer, stream, randn, steps):
    """Config 1: FP32 GEMV x[1,1024] . W[1024->3584], 36 rotating copies (528 MB)."""
    extra = {}
    ws = []
    for _ in range(36):
        w = randn(I, H, std=0.02, dtype=torch.float32)
        ws.append(qw.Weight.pack_device(ctx, w, qw.WFMT_F32))
        del w
    x1 = randn(1, H, dtype=torch.float32)
    y1 = torch.empty(1, I, device="cuda")
    g = graphed(qw, ctx, stream, lambda: [qw.linear(ctx, w, x1, y1) for w in ws])
    ms = timer.run(g.launch, steps, 2)
    b = 36 * (I * H * 4 + H * 4 + I * 4)
    extra["cfg1_gemv_f32_M1"] = {"us_per_gemv": round(ms * 1e3 / 36, 2), "GBps": round(b / ms / 1e6, 1),
                                 "pct_hbm": round(100 * b / ms / 1e6 / HBM_PEAK, 1)}
    log("cfg1", extra["cfg1_gemv_f32_M1"])
    del ws, g
    return extra


def run_cfg3(qw, ctx, torch, timer, stream, randn, steps):
    """Config 3: INT8 weight-only projections of all 24 layers, FP16 activations."""
    extra = {}

    # config 3: INT8 weight-only projections of all 24 layers, FP16 activations
    def i8(n, k):
        q = torch.randint(-127, 128, (n, k), generator=torch.Generator(device="cuda").manual_seed(n * 7 + k),
                          device="cuda", dtype=torch.int8)
        s = torch.rand(n, generator=torch.Generator(device="cuda").manual_seed(n + k), device="cuda") * (2e-2 - 1e-3) + 1e-3
        return q, s

    # Projections that read the same activation are stacked into one weight
    # (qw_weight_pack_concat): QKV+Z of a Gated-DeltaNet layer, Q+gate/K/V of
    # a full-attention layer -- one launch each.
    layers = []
    wbytes = 0
    for li in range(LAYERS):
        L = {}
        if li in LINEAR_LAYERS:
            ins = [(6144, 1024), (2048, 1024)]
        else:
            ins = [(4096, 1024), (512, 1024), (512, 1024)]
        qs, ss = zip(*[i8(n, k) for n, k in ins])
        L["in"] = qw.Weight.pack_concat_device(ctx, list(qs), qw.WFMT_INT8, scales=list(ss))
        L["n_in"] = sum(n for n, _ in ins)
        wbytes += sum(n * k + n * 4 for n, k in ins)
        q, s_ = i8(1024, 2048)
        L["out"] = qw.Weight.pack_device(ctx, q, qw.WFMT_INT8, scales=s_)
        wbytes += 1024 * 2048 + 1024 * 4
        del qs, ss
        qg_, sg_ = i8(I, H)
        qu_, su_ = i8(I, H)
        L["gu"] = qw.Weight.pack_glu_device(ctx, qg_, qu_, qw.WFMT_INT8, sg_, su_)
        qd_, sd_ = i8(H, I)
        L["down"] = qw.Weight.pack_device(ctx, qd_, qw.WFMT_INT8, scales=sd_)
        wbytes += 3 * H * I + 2 * I * 4 + H * 4
        layers.append(L)
    torch.cuda.synchronize()
    for M in (1, 32, 128):
        xa = randn(M, H, dtype=torch.float16)
        att = randn(M, 2048, dtype=torch.float16)            # attention-core stand-in
        big = torch.empty(M, 8192, device="cuda", dtype=torch.float16)
        res = randn(M, H, dtype=torch.float16)

        def body():
            for L in layers:
                qw.linear(ctx, L["in"], xa, big[:, :L["n_in"]])
                qw.linear(ctx, L["out"], att, res, residual=res)
                # the MLP block: one launch at M <= 16, else gate/up then down
                qw.mlp_fused(ctx, L["gu"], L["down"], xa, res, residual=res)
        g = graphed(qw, ctx, stream, body)
        ms = timer.run(g.launch, steps, 2)
        act = 0
        for li in range(LAYERS):
            if li in LINEAR_LAYERS:
                act += M * 2 * (1024 * 3 + 6144 + 2048 + 2048 + 1024 * 3)
            else:
                act += M * 2 * (1024 * 3 + 4096 + 512 * 2 + 2048 + 1024 * 3)
            act += M * 2 * (1024 + 2 * I + I + 1024)
        b = wbytes + act
        fl = 2.0 * M * (wbytes)  # one MAC per weight byte
        extra[f"cfg3_int8_stack_M{M}"] = {"us_per_step": round(ms * 1e3, 1), "GBps": round(b / ms / 1e6, 1),
                                          "pct_hbm": round(100 * b / ms / 1e6 / HBM_PEAK, 1),
                                          "TFLOPs": round(fl / ms / 1e9, 2)}
        log("cfg3", M, extra[f"cfg3_int8_stack_M{M}"])
        del g
    # The config-3 MLP blocks alone (INT8 gate/up and down, F16 activations,
    # per-call RMSNorm weight) as one persistent qw_mlp_stack launch.
    gams = [randn(H, std=0.02, dtype=torch.float32) for _ in range(LAYERS)]
    for M in (1, 8):
        xs = randn(M, H, dtype=torch.float16)
        g = graphed(qw, ctx, stream, lambda xs=xs: qw.mlp_stack(ctx, [L["gu"] for L in layers],
                                                                [L["down"] for L in layers], xs, xs, gammas=gams,
                                                                stream=stream))
        ms = timer.run(g.launch, steps, 2)
        if ctx.device_error():
            raise RuntimeError("device error flag after the INT8 MLP stack")
        b = LAYERS * (3 * H * I + (2 * I + H) * 4 + M * H * 2 * 2 + H * 4)
        extra[f"cfg3_int8_mlp_stack_M{M}"] = {"us_per_layer": round(ms * 1e3 / LAYERS, 2),
                                              "GBps": round(b / ms / 1e6, 1),
                                              "pct_hbm": round(100 * b / ms / 1e6 / HBM_PEAK, 1)}
        log("cfg3 int8 mlp stack", M, extra[f"cfg3_int8_mlp_stack_M{M}"])
        del g
    # The same 24 layers as ONE persistent projection chain (qw_chain) at
    # decode sizes, in the model's dependency order: in -> out (reading the
    # first 2048 outputs of in, the attention core's stand-in) + residual ->
    # gate/up -> down + residual -> the next layer's in.
    for M in (1, 2):
        xa = randn(M, H, dtype=torch.float16)
        xo = torch.empty(M, H, device="cuda", dtype=torch.float16)
        slots = [{"len": H, "init": xa, "out": xo}, {"len": 8192}, {"len": I}]
        ops = []
        for L in layers:
            ops += [{"w": L["in"], "in": 0, "out": 1}, {"w": L["out"], "in": 1, "out": 0, "residual": True},
                    {"w": L["gu"], "in": 0, "out": 2}, {"w": L["down"], "in": 2, "out": 0, "residual": True}]
        ch = qw.Chain(ctx, qw.F16, M, slots, ops)
        g = graphed(qw, ctx, stream, lambda: ch.launch(stream))
        ms = timer.run(g.launch, steps, 2)
        if ctx.device_error():
            raise RuntimeError("device error flag after the projection chain")
        act = 0
        for li in range(LAYERS):
            n_in = 8192 if li in LINEAR_LAYERS else 5120
            act += M * 2 * (1024 + n_in + 2048 + 1024 * 2 + 1024 + I + I + 1024 * 2)
        b = wbytes + act
        extra[f"cfg3_int8_chain_M{M}"] = {"us_per_step": round(ms * 1e3, 1), "GBps": round(b / ms / 1e6, 1),
                                          "pct_hbm": round(100 * b / ms / 1e6 / HBM_PEAK, 1),
                                          "launches": 1, "ops": len(ops)}
        log("cfg3 chain", M, extra[f"cfg3_int8_chain_M{M}"])
        del g
        ch.close()
    del layers

    return extra


def run_int8_gemv(qw, ctx, torch, timer, stream, randn, steps):
    """The north star's own kernel line: one INT8 weight-only decode GEMV at
    M=1 (x[1,1024] F16 times an INT8 W[3584,1024] with per-row scales), 80
    distinct weights (294 MB, beyond the 256 MB Infinity Cache) replayed from
    a graph, so every launch streams its 3.67 MB from HBM; and the same for
    the gate/up GLU pair (7.3 MB per launch, SiLU*mul fused)."""
    out = {}
    n_copies = 80

    def i8(n, k, seed):
        q = torch.randint(-127, 128, (n, k), generator=torch.Generator(device="cuda").manual_seed(seed),
                          device="cuda", dtype=torch.int8)
        s = torch.rand(n, generator=torch.Generator(device="cuda").manual_seed(seed + 1), device="cuda") * 1e-3 + 1e-4
        return q, s

    x = randn(1, H, dtype=torch.float16)
    ws = []
    for c in range(n_copies):
        q, s_ = i8(I, H, 7000 + 2 * c)
        ws.append(qw.Weight.pack_device(ctx, q, qw.WFMT_INT8, scales=s_))
    y = torch.empty(1, I, device="cuda", dtype=torch.float16)
    g = graphed(qw, ctx, stream, lambda: [qw.linear(ctx, w, x, y) for w in ws])
    us = 1e3 * timer.run(g.launch, max(5, steps), 2) / n_copies
    b = I * H + I * 4 + H * 2 + I * 2
    out["int8_gemv_3584x1024_M1"] = {"us_per_launch": round(us, 3), "GBps": round(b / us / 1e3, 1),
                                     "pct_hbm": round(100 * b / us / 1e3 / HBM_PEAK, 1), "bytes_per_launch": b}
    log("int8 gemv", out["int8_gemv_3584x1024_M1"])
    del g, ws
    gus = []
    for c in range(n_copies // 2):
        qg, sg = i8(I, H, 8000 + 4 * c)
        qu, su = i8(I, H, 8002 + 4 * c)
        gus.append(qw.Weight.pack_glu_device(ctx, qg, qu, qw.WFMT_INT8, sg, su))
    g = graphed(qw, ctx, stream, lambda: [qw.linear(ctx, w, x, y) for w in gus])
    us = 1e3 * timer.run(g.launch, max(5, steps), 2) / len(gus)
    b = 2 * I * H + 2 * I * 4 + H * 2 + I * 2
    out["int8_gemv_gateup_glu_M1"] = {"us_per_launch": round(us, 3), "GBps": round(b / us / 1e3, 1),
                                      "pct_hbm": round(100 * b / us / 1e3 / HBM_PEAK, 1), "bytes_per_launch": b}
    log("int8 gemv glu", out["int8_gemv_gateup_glu_M1"])
    del g, gus
    return out


def run_wide(qw, ctx, torch, timer, stream, randn, steps):
    """Per-launch lines of the weight-stationary kernel (qw_wide.hip) at 32 and
    128 tokens: the gate/up GLU pair (BF16 and INT8) and the down projection
    with the residual, 24 distinct weights per graph so every launch streams
    its weights from HBM."""
    out = {}
    n_copies = 24
    for fmt in ("bf16", "int8"):
        wf = qw.WFMT_BF16 if fmt == "bf16" else qw.WFMT_INT8
        xdt = torch.bfloat16 if fmt == "bf16" else torch.float16
        wb = 2 if fmt == "bf16" else 1

        def mk(n, k, seed):
            if fmt == "bf16":
                return randn(n, k, std=0.02), None
            q = torch.randint(-127, 128, (n, k), generator=torch.Generator(device="cuda").manual_seed(seed),
                              device="cuda", dtype=torch.int8)
            return q, torch.rand(n, generator=torch.Generator(device="cuda").manual_seed(seed + 1),
                                 device="cuda") * 1e-3 + 1e-4

        gus, dns = [], []
        for c in range(n_copies):
            (a_, sa), (b_, sb) = mk(I, H, 9000 + 4 * c), mk(I, H, 9002 + 4 * c)
            gus.append(qw.Weight.pack_glu_device(ctx, a_, b_, wf, sa, sb))
            d_, sd = mk(H, I, 9500 + 2 * c)
            dns.append(qw.Weight.pack_device(ctx, d_, wf, scales=sd))
        for M in (32, 128):
            x = randn(M, H, dtype=xdt)
            h = torch.empty(M, I, device="cuda", dtype=xdt)
            r = randn(M, H, dtype=xdt)
            g = graphed(qw, ctx, stream, lambda: [qw.linear(ctx, w, x, h) for w in gus])
            us = 1e3 * timer.run(g.launch, max(5, steps), 2) / n_copies
            b = 2 * I * H * wb + (2 * I * 4 if fmt == "int8" else 0) + M * H * 2 + M * I * 2
            out[f"wide_gateup_{fmt}_M{M}"] = {"us_per_launch": round(us, 3), "GBps": round(b / us / 1e3, 1),
                                              "pct_hbm": round(100 * b / us / 1e3 / HBM_PEAK, 1),
                                              "bytes_per_launch": b}
            log("wide", fmt, M, out[f"wide_gateup_{fmt}_M{M}"])
            del g
            g = graphed(qw, ctx, stream, lambda: [qw.linear(ctx, w, h, r, residual=r) for w in dns])
            us = 1e3 * timer.run(g.launch, max(5, steps), 2) / n_copies
            b = H * I * wb + (H * 4 if fmt == "int8" else 0) + M * I * 2 + 2 * M * H * 2
            out[f"wide_down_{fmt}_M{M}"] = {"us_per_launch": round(us, 3), "GBps": round(b / us / 1e3, 1),
                                            "pct_hbm": round(100 * b / us / 1e3 / HBM_PEAK, 1),
                                            "bytes_per_launch": b}
            log("wide", fmt, M, out[f"wide_down_{fmt}_M{M}"])
            del g
        del gus, dns
    return out


def run_lmhead(qw, ctx, torch, timer, stream, randn, steps):
    """Config 5: tied lm_head + greedy argmax, BF16 and INT8, 2 rotating copies each."""
    extra = {}
    for fmt, name in ((qw.WFMT_BF16, "bf16"), (qw.WFMT_INT8, "int8")):
        Es = []
        for c in range(2):
            e = randn(V, H, std=0.02)
            Es.append(qw.Weight.pack_device(ctx, e, fmt))
            del e
        torch.cuda.synchronize()
        wb = V * H * (2 if fmt == qw.WFMT_BF16 else 1) + (V * 4 if fmt == qw.WFMT_INT8 else 0)
        for M in (1, 32, 128):
            hh = randn(M, H)
            ids = torch.empty(M, dtype=torch.int32, device="cuda")
            g = graphed(qw, ctx, stream, lambda hh=hh, ids=ids: [qw.lmhead_argmax(ctx, E, hh, ids) for E in Es])
            ms = timer.run(g.launch, max(3, steps // 4), 1) / 2
            b = wb + M * H * 2 + M * 4
            extra[f"cfg5_lmhead_{name}_M{M}"] = {"us_per_call": round(ms * 1e3, 1), "GBps": round(b / ms / 1e6, 1),
                                                 "pct_hbm": round(100 * b / ms / 1e6 / HBM_PEAK, 1),
                                                 "tok_per_s": round(M / (ms * 1e-3), 1)}
            log("cfg5", name, M, extra[f"cfg5_lmhead_{name}_M{M}"])
            del g
        del Es
    torch.cuda.synchronize()
    return extra


def run_decode_model(qw, ctx, torch, timer, stream, randn, args, b1_only=False):
    """The whole greedy decode step of the 24-layer model (engine.py: embedding
    gather, 18 Gated-DeltaNet + 6 full-attention layers, fused MLPs, final norm,
    lm_head argmax over 248320 tokens, position advance) captured as one graph
    and replayed per token; BF16 weights (random init, real shapes), INT8 KV
    cache, B sequences at a context of 1024 tokens (random cache contents and
    recurrent states).  Then the whole-model prefill of 1024-token prompts."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("qw_engine", os.path.join(os.path.dirname(os.path.abspath(__file__)), "qwen3.5_0.8b_deploy_amd", "engine.py"))
    em = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(em)
    f32 = torch.float32
    layers = []
    for i in range(LAYERS):
        L = {"in_norm": randn(H, std=0.1, dtype=f32), "post_norm": randn(H, std=0.1, dtype=f32),
             "gate": randn(I, H, std=0.02, dtype=f32), "up": randn(I, H, std=0.02, dtype=f32),
             "down": randn(H, I, std=0.02, dtype=f32)}
        if em.is_linear_layer(i):
            L.update(qkv=randn(em.CD, H, std=0.02, dtype=f32), a=randn(em.LNH, H, std=0.02, dtype=f32),
                     b=randn(em.LNH, H, std=0.02, dtype=f32), z=randn(em.LNH * em.VD, H, std=0.02, dtype=f32),
                     conv=randn(em.CD, em.CK, std=0.5, dtype=f32), out=randn(H, em.LNH * em.VD, std=0.02, dtype=f32),
                     A_log=randn(em.LNH, std=0.5, dtype=f32), dt_bias=randn(em.LNH, std=0.5, dtype=f32),
                     norm_w=1.0 + randn(em.VD, std=0.1, dtype=f32))
        else:
            L.update(q=randn(em.FNH * 2 * em.HD, H, std=0.02, dtype=f32), k=randn(em.FNKV * em.HD, H, std=0.02, dtype=f32),
                     v=randn(em.FNKV * em.HD, H, std=0.02, dtype=f32), q_norm=randn(em.HD, std=0.1, dtype=f32),
                     k_norm=randn(em.HD, std=0.1, dtype=f32), o=randn(H, em.FNH * em.HD, std=0.02, dtype=f32))
        layers.append(L)
    embed = randn(V, H, std=0.02)  # BF16 table, tied with the lm_head
    final_norm = randn(H, std=0.1, dtype=f32)
    out = {}
    ctxlen = 1024
    for B in ((1,) if b1_only else (1, 32)):
        eng = em.DecodeEngine(qw, ctx, layers, final_norm, embed, B, ctxlen + 256)
        eng.reset(torch.randint(0, V, (B,)).tolist(), [ctxlen] * B)
        for P in eng.layers:
            if P["linear"]:
                P["rs"].normal_(0.0, 0.1)
            else:
                P["cache"][0].random_(-127, 128)
                P["cache"][1].random_(-127, 128)
                P["cache"][2].uniform_(0.001, 0.01)
                P["cache"][3].uniform_(0.001, 0.01)
        g = graphed(qw, ctx, stream, lambda: eng.step(stream=stream))
        n = max(8, args.steps)
        ms = timer.run(g.launch, n, 2)
        out[f"decode_model_B{B}_ctx{ctxlen}"] = {"ms_per_step": round(ms, 3), "tok_per_s": round(B / (ms * 1e-3), 1)}
        log("decode model", B, out[f"decode_model_B{B}_ctx{ctxlen}"])
        del eng, g
    # whole-model prefill of a T-token prompt per sequence (engine.prefill:
    # embedding, 24 layers with M = B*T rows, final norm, next-token argmax),
    # from position 0 with cleared states; the reset is outside the timed
    # region.  T=512 at B=1 is a mid-size prompt, where the 1024-row
    # projections sit between the small-M kernels and the split-K GEMM
    for B, T in (() if b1_only else ((1, 1024), (16, 1024), (1, 512))):
        eng = em.DecodeEngine(qw, ctx, layers, final_norm, embed, B, T + 256)
        prompt = torch.randint(0, V, (B, T), device="cuda", dtype=torch.int32)
        times = []
        with torch.cuda.stream(stream):
            for it in range(4):
                eng.reset([0] * B)
                torch.cuda.synchronize()
                t0 = torch.cuda.Event(enable_timing=True)
                t1 = torch.cuda.Event(enable_timing=True)
                t0.record(stream)
                eng.prefill(prompt, stream=stream)
                t1.record(stream)
                torch.cuda.synchronize()
                if it:  # the first pass warms up
                    times.append(t0.elapsed_time(t1))
        ms = sorted(times)[len(times) // 2]
        out[f"prefill_model_B{B}_T{T}"] = {"ms": round(ms, 3), "tok_per_s": round(B * T / (ms * 1e-3), 1)}
        log("prefill model", B, T, out[f"prefill_model_B{B}_T{T}"])
        del eng
    del layers, embed
    torch.cuda.empty_cache()
    return out


def run_attn(qw, ctx, torch, timer, stream, randn, args):
    """Gated full attention between the projections (6 of the 24 layers): the
    norm/RoPE/cache-write prep, causal attention over the INT8 KV cache and
    the gate, for (a) decode steps of B sequences at a context of L tokens and
    (b) a T-token prefill of one sequence.  Decode bytes: the K and V codes
    and scales of the context (2 x L x 2 heads x (256 + 4) per sequence)."""
    NH, NKV, HD = 8, 2, 256
    LD = NH * 2 * HD + 2 * NKV * HD
    qn = 0.1 * randn(HD, dtype=torch.float32)
    kn = 0.1 * randn(HD, dtype=torch.float32)
    out = {}

    def call(cache, rows, pos, tokens, o, max_len):
        qw.attn_forward(ctx, qn, kn, cache, pos, rows[:, 0:], rows[:, HD:], rows[:, NH * 2 * HD:],
                        rows[:, NH * 2 * HD + NKV * HD:], o, tokens=tokens, q_head_stride=2 * HD, max_len=max_len)

    for B, L in ((1, 512), (1, 4096), (1, 32768), (32, 4096)):
        cache = qw.kv_cache(B, L + 1)
        cache[0].random_(-127, 128)
        cache[1].random_(-127, 128)
        cache[2].uniform_(0.001, 0.01)
        cache[3].uniform_(0.001, 0.01)
        rows = randn(B, LD, dtype=torch.float32)
        pos = torch.full((B,), L, dtype=torch.int32, device="cuda")
        o = torch.empty(B, NH * HD, device="cuda", dtype=torch.bfloat16)
        g = graphed(qw, ctx, stream, lambda: call(cache, rows, pos, 1, o, L + 1))
        us = 1e3 * timer.run(g.launch, max(5, args.steps // 2), 2)
        by = B * 2 * (L + 1) * NKV * (HD + 4)
        out[f"attn_decode_B{B}_L{L}"] = {"us_per_layer": round(us, 2), "GBps": round(by / us / 1e3, 1),
                                         "pct_hbm": round(100 * by / us / 1e3 / HBM_PEAK, 1)}
        log("attn decode", B, L, out[f"attn_decode_B{B}_L{L}"])
        del cache, g
    for T in (1024, 4096):
        cache = qw.kv_cache(1, T)
        rows = randn(T, LD, dtype=torch.float32)
        pos = torch.zeros(1, dtype=torch.int32, device="cuda")
        o = torch.empty(T, NH * HD, device="cuda", dtype=torch.bfloat16)
        ms = timer.run(lambda: call(cache, rows, pos, T, o, T), 3, 1)
        flops = 2 * 2 * NH * HD * T * (T + 1) / 2  # QK^T and PV over the causal triangle
        out[f"attn_prefill_T{T}"] = {"us_per_layer": round(1e3 * ms, 1), "TFLOPs": round(flops / ms / 1e9, 1)}
        log("attn prefill", T, out[f"attn_prefill_T{T}"])
        del cache
    return out


def run_gdn(qw, ctx, torch, timer, stream, randn, args):
    """Gated-DeltaNet decode (the next row after the projections): one token
    of each of B sequences through the 18 linear-attention layers, (a) the
    step between the projections alone (conv1d, gates, delta rule on the FP32
    state, norm-gate), and (b) the whole layer: the stacked QKV+Z+a+b
    projection (FP32 out), the step (BF16 out), the out projection with the
    residual add.  BF16 weights.  Bytes: the state is read and written
    (2 x 16 x 128 x 128 x 4 per sequence) plus the conv state; the layer adds
    its weights (8224 x 1024 + 1024 x 2048, BF16)."""
    NH, KD, VD, K = 16, 128, 128, 4
    CD = 2 * NH * KD + NH * VD
    NIN = CD + NH * VD + 2 * NH
    layers = []
    for li in range(len(LINEAR_LAYERS)):
        parts = [randn(n, H, std=0.02) for n in (CD, NH * VD, NH, NH)]
        L = {"in": qw.Weight.pack_concat_device(ctx, parts, qw.WFMT_BF16)}
        del parts
        o = randn(H, NH * VD, std=0.02)
        L["out"] = qw.Weight.pack_device(ctx, o, qw.WFMT_BF16)
        del o
        L["conv_w"] = randn(CD, K, std=0.5, dtype=torch.float32)
        L["A_log"] = randn(NH, std=0.5, dtype=torch.float32)
        L["dt_bias"] = randn(NH, std=0.5, dtype=torch.float32)
        L["norm_w"] = 1.0 + randn(VD, std=0.1, dtype=torch.float32)
        layers.append(L)
    out = {}
    for B in (1, 32):
        x = randn(B, H)
        res = randn(B, H)
        row = torch.empty(B, NIN, device="cuda", dtype=torch.float32)
        core = torch.empty(B, NH * VD, device="cuda", dtype=torch.bfloat16)
        for L in layers:
            L["cs"] = torch.zeros(B, CD, K - 1, device="cuda")
            L["rs"] = randn(B, NH, KD * VD, std=0.1, dtype=torch.float32)
        qw.linear(ctx, layers[0]["in"], x, row)
        torch.cuda.synchronize()

        def step(L):
            qw.gdn_decode(ctx, L["conv_w"], L["A_log"], L["dt_bias"], L["norm_w"], row[:, :CD],
                          row[:, CD:CD + NH * VD], row[:, CD + NH * VD:CD + NH * VD + NH],
                          row[:, CD + NH * VD + NH:], L["cs"], L["rs"], core, NH)

        def layer_body():
            for L in layers:
                qw.linear(ctx, L["in"], x, row)
                step(L)
                qw.linear(ctx, L["out"], core, res, residual=res)

        g1 = graphed(qw, ctx, stream, lambda: [step(L) for L in layers])
        us = 1e3 * timer.run(g1.launch, max(3, args.steps // 5), 1) / len(layers)
        sb = B * (NH * KD * VD * 4 * 2 + CD * (K - 1) * 4 * 2)
        out[f"gdn_step_B{B}"] = {"us_per_layer": round(us, 2), "GBps": round(sb / us / 1e3, 1),
                                 "pct_hbm": round(100 * sb / us / 1e3 / HBM_PEAK, 1)}
        g2 = graphed(qw, ctx, stream, layer_body)
        us2 = 1e3 * timer.run(g2.launch, max(3, args.steps // 5), 1) / len(layers)
        lb = sb + (NIN * H + H * NH * VD) * 2
        out[f"gdn_layer_decode_B{B}"] = {"us_per_layer": round(us2, 2), "GBps": round(lb / us2 / 1e3, 1),
                                         "tok_per_s_18_layers": round(B / (us2 * len(layers) * 1e-6), 1)}
        log("gdn", B, out[f"gdn_step_B{B}"], out[f"gdn_layer_decode_B{B}"])
        del g1, g2
    # prefill of one sequence: T tokens serially through the recurrence (one launch per layer)
    T = 1024
    rows = randn(T, NIN, dtype=torch.float32)
    core = torch.empty(T, NH * VD, device="cuda", dtype=torch.bfloat16)
    L = layers[0]
    cs = torch.zeros(1, CD, K - 1, device="cuda")
    rs = torch.zeros(1, NH, KD * VD, device="cuda")

    def pre():
        qw.gdn_prefill(ctx, L["conv_w"], L["A_log"], L["dt_bias"], L["norm_w"], rows[:, :CD],
                       rows[:, CD:CD + NH * VD], rows[:, CD + NH * VD:CD + NH * VD + NH], rows[:, CD + NH * VD + NH:],
                       cs, rs, core, NH, T)
    ms = timer.run(pre, 3, 1)
    out[f"gdn_prefill_T{T}"] = {"us_per_layer": round(1e3 * ms, 1), "tok_per_s_per_layer": round(T / (ms * 1e-3), 0)}
    log("gdn prefill", out[f"gdn_prefill_T{T}"])
    del layers
    return out


def run_prefill(qw, ctx, torch, timer, stream, randn, args, M=16384):
    """Config 4: the 24-layer BF16 projection stack at M=16384 prefill tokens.

    Per Gated-DeltaNet layer: QKV 1024->6144 and Z 1024->2048 (one stacked
    weight), out 2048->1024 (+residual); per full-attention layer: Q+gate
    1024->4096, K and V 1024->512 (one stacked weight), O 2048->1024
    (+residual); every layer: RMSNorm + gate/up 1024->2x3584 with SiLU*mul,
    down 3584->1024 (+residual).  The attention
    cores between the projections are outside this path; a fixed [M][2048]
    tensor stands in for their output.  FLOPs = 2*M*sum(N*K) = 16.29 TFLOP."""
    ws = []
    nk = 0
    for li in range(LAYERS):
        L = {}
        # the input projections of a layer share x: one stacked weight per
        # layer (qw_weight_pack_concat), as the loader packs them
        if li in LINEAR_LAYERS:
            ins, out_k = [(6144, 1024), (2048, 1024)], 2048
        else:
            ins, out_k = [(4096, 1024), (512, 1024), (512, 1024)], 2048
        parts = [randn(n, k, std=0.02) for n, k in ins]
        L["in"] = qw.Weight.pack_concat_device(ctx, parts, qw.WFMT_BF16)
        L["n_in"] = sum(n for n, _ in ins)
        nk += sum(n * k for n, k in ins)
        del parts
        o = randn(1024, out_k, std=0.02)
        L["out"] = qw.Weight.pack_device(ctx, o, qw.WFMT_BF16)
        nk += 1024 * out_k
        del o
        g, u = randn(I, H, std=0.02), randn(I, H, std=0.02)
        L["gu"] = qw.Weight.pack_glu_device(ctx, g, u, qw.WFMT_BF16)
        d = randn(H, I, std=0.02)
        L["down"] = qw.Weight.pack_device(ctx, d, qw.WFMT_BF16)
        L["gamma"] = randn(H, std=0.02, dtype=torch.float32)
        nk += 3 * H * I
        del g, u, d
        ws.append(L)
    x = randn(M, H)
    att = randn(M, 2048)
    big = torch.empty(M, 8192, device="cuda", dtype=torch.bfloat16)
    hmid = torch.empty(M, I, device="cuda", dtype=torch.bfloat16)
    res = randn(M, H)
    torch.cuda.synchronize()

    def body():
        for L in ws:
            qw.linear(ctx, L["in"], x, big[:, :L["n_in"]], ldy=8192)
            qw.linear(ctx, L["out"], att, res, residual=res)
            qw.linear(ctx, L["gu"], res, hmid, gamma=L["gamma"])
            qw.linear(ctx, L["down"], hmid, res, residual=res)

    ms = timer.run(body, max(3, args.steps // 10), 1)
    fl = 2.0 * M * nk
    out = {"cfg4_prefill_bf16_M16384": {"ms_per_stack": round(ms, 3), "TFLOPs": round(fl / ms / 1e9, 1),
                                        "pct_mfma_peak": round(100 * fl / ms / 1e9 / BF16_PEAK, 1),
                                        "tok_per_s": round(M / (ms * 1e-3), 1), "sum_NK": nk}}
    log("cfg4", out)
    del ws
    return out


if __name__ == "__main__":
    main()
