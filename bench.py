#!/usr/bin/env python3
"""Benchmark of the MI355X q4 x int8 matmul path (libkq4) on BASELINE.json's workload.

Workload: the full decode-step linear set of a Qwen3-VL-2B-shaped
decoder - QKV (2048 -> 16 q + 8 kv heads x 128, one fused launch), O (2048 -> 2048, + residual),
gate/up (2048 -> 6144, one fused launch) and down (6144 -> 2048, + residual) - for all 28
layers, at M = 1 token (--m 4 for the config's second batch). One step = one token through the
28 layers' linear sets: 4 launches per layer (each quantizes its activations and multiplies),
captured once as a HIP graph and replayed per step; the eager (host-launched) time is reported
beside it. The 28 layers are distinct HBM copies (28 x 28.3 MB = 793 MB > the 256 MB Infinity
Cache), so every step streams its weights from HBM. Inputs are resident in HBM before the timed
region.

value = algorithmic bytes per step (weights N*K*18/32 + activations M*K*4 + outputs M*N*4 +
residuals M*N*4) / step time, in GB/s. roofline: the dominant kernel (the fused gate/up GEMV,
launched exactly as in the step, once per layer's weights), its launches captured back to back
as a graph and replayed between HIP events on their stream, against MI355X HBM peak 8 TB/s.
extras: the other BASELINE.json configs, each with a roofline block per op (config 1 single
GEMV, config 2 at M = 4, Qwen3-8B decode GEMVs, prefill GEMM against int8 dense peak, MoE FFN).
cpu_baseline: the reference's own x86-64 code for every config (oracle/cpu_bench.py over
oracle/_ref, built from /root/reference): median of >= 20 reps at all physical cores and at
the reference's default thread count.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--m 1] [--no-cpu] [--no-extras]
    python bench.py --calibrate-copy      (512 MiB copy for PMC byte-counter scaling)
    python bench.py --profile-op OP --m M --reps R   (one op repeated, for rocprofv3 runs)
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kestrel-llm_amd"))

import numpy as np  # noqa: E402

import synth  # noqa: E402

METRIC = "q4 GEMV µs/call + HBM GB/s (% peak); prefill GEMM int8 TOPS (% peak)"
HBM_PEAK_GBS = 8000.0
CFG = synth.QWEN3VL_2B


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "pmc_hbm_traffic_gemv_qwen3vl2b_m1.md")


def profiled_traffic(m):
    """HBM bytes per launch of the dominant kernel at M = 1, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (copy-calibrated), and the commit of the kernel sources it
    was measured on (the summary's `measured_at_commit:` line); (None, None) for other M or
    without it. The counters cannot be read inside a timed run, so the figure is only as current
    as that commit."""
    if m != 1:
        return None, None
    byts = commit = None
    try:
        with open(TRAFFIC_PROFILE) as fh:
            for line in fh:
                if line.startswith("traffic_bytes_per_launch:"):
                    byts = int(line.split(":")[1])
                elif line.startswith("measured_at_commit:"):
                    commit = line.split(":")[1].strip()
    except OSError:
        pass
    return byts, commit


def layer_mats():
    return {name: (rows, cols) for name, rows, cols in synth.layer_shapes(CFG)}


def step_bytes(m):
    """Algorithmic bytes of one layer's linear set at m tokens (x counted once per launch)."""
    s = layer_mats()
    wb = sum(r * c * 18 // 32 for r, c in s.values())
    h, q, kv, f = CFG["hidden"], s["q"][0], s["k"][0], CFG["ffn"]
    act = m * 4 * (h + q + h + f)                     # x of QKV, O, gate/up, down
    out = m * 4 * (q + 2 * kv + h + 2 * f + h)
    res = m * 4 * (h + h)                             # residual reads of O and down
    return wb + act + out + res


def gate_up_bytes(m):
    h, f = CFG["hidden"], CFG["ffn"]
    return 2 * f * h * 18 // 32 + m * h * 4 + 2 * m * f * 4


def make_model(torch, n_layers, seed=1):
    """One layer of seeded weights (device copies in the stream layout), copied to n_layers
    distinct HBM buffers."""
    import kq4
    mats = layer_mats()
    base = {name: synth.make_q4_weights(r, c, seed + i, **synth.SCALE_2B)
            for i, (name, (r, c)) in enumerate(mats.items())}
    dev0 = {k: kq4.prepare_dev(torch.from_numpy(v.reshape(-1)).cuda(), *mats[k])
            for k, v in base.items()}
    return [{k: v.clone() for k, v in dev0.items()} for _ in range(n_layers)], base


def run_gpu(args):
    import torch

    import kq4

    kq4.init(0)
    torch.cuda.set_device(0)
    m = args.m
    s = layer_mats()
    h, q, kv, f = CFG["hidden"], s["q"][0], s["k"][0], CFG["ffn"]
    layers, _ = make_model(torch, CFG["layers"])
    dev = lambda shape: torch.empty(shape, dtype=torch.float32, device="cuda")  # noqa: E731
    x = torch.from_numpy(synth.make_activations(m, h, 7)).cuda()
    attn = torch.from_numpy(synth.make_activations(m, q, 8)).cuda()
    act = torch.from_numpy(synth.make_activations(m, f, 9)).cuda()
    resid = torch.from_numpy(synth.make_activations(m, h, 10)).cuda()
    oq, ok_, ov, oo, og, ou, od = dev((m, q)), dev((m, kv)), dev((m, kv)), dev((m, h)), \
        dev((m, f)), dev((m, f)), dev((m, h))

    def layer_ops(L, st):
        kq4.matmul_multi_dev([oq, ok_, ov], x, [L["q"], L["k"], L["v"]], [q, kv, kv], h,
                             stream=st)
        kq4.matmul_dev(oo, attn, L["o"], h, q, residual=resid, stream=st)
        kq4.matmul_multi_dev([og, ou], x, [L["gate"], L["up"]], [f, f], h, stream=st)
        kq4.matmul_dev(od, act, L["down"], h, f, residual=resid, stream=st)

    def step():
        st = torch.cuda.current_stream()
        for L in layers:
            layer_ops(L, st)

    def timed(fn, k):
        torch.cuda.synchronize()
        st = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(k):
            fn()
        e1.record(st)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / k

    # eager: one host launch per op (4 per layer)
    for _ in range(args.warmup):
        step()
    ms_eager = timed(step, args.steps)

    # the same step captured once as a HIP graph and replayed (how a decode loop runs it)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(args.warmup):
        graph.replay()
    ms_graph = timed(graph.replay, args.steps)
    total_bytes = step_bytes(m) * CFG["layers"]

    # dominant kernel: the fused gate/up GEMV launch exactly as the step issues it, one per
    # layer's weights, captured as a graph of back-to-back launches and replayed between HIP
    # events recorded on the stream the launches run on
    st = torch.cuda.current_stream()
    gu = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gu):
        for L in layers:
            kq4.matmul_multi_dev([og, ou], x, [L["gate"], L["up"]], [f, f], h,
                                 stream=torch.cuda.current_stream())
    gu.replay()
    reps = max(4, args.steps // 4)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        gu.replay()
    e1.record(st)
    torch.cuda.synchronize()
    us_launch = e0.elapsed_time(e1) * 1e3 / (reps * len(layers))
    achieved = gate_up_bytes(m) / (us_launch * 1e-6) / 1e9
    return dict(ms_per_step=ms_graph, ms_eager=ms_eager,
                value=total_bytes / (ms_graph * 1e-3) / 1e9,
                value_eager=total_bytes / (ms_eager * 1e-3) / 1e9,
                us_gate_up=us_launch, achieved=achieved, total_bytes=total_bytes)


def copy_calibration(mib=512, reps=10):
    """A plain device-to-device copy of known size, for scaling rocprofv3 FETCH_SIZE /
    WRITE_SIZE counters to bytes (run under --pmc; its kernel reads and writes exactly
    `mib` MiB per launch)."""
    import torch

    n = mib * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    return dict(copy_mib=mib, reps=reps)


def _time_graph(torch, fn, n, reps=5, warm_ms=20.0):
    """Average us per call of fn(0..n-1) (one call per rotated weight copy): the n calls are
    captured as one HIP graph and replayed reps times between events on the capture stream, so
    no host launch cost is in the timed region. An eager pass first sizes the library's
    workspaces and touches every copy; untimed replays for at least warm_ms then let the clock
    settle under the load (the first milliseconds of a heavy graph after lighter work run up to
    ~15 % slower)."""
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        for i in range(n):
            fn(i, st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        for i in range(n):
            fn(i, st)
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(1000):
        if (time.perf_counter() - t0) * 1e3 >= warm_ms:
            break
        g.replay()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        with torch.cuda.stream(st):
            g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * n)


ROTATE_BYTES = 640e6   # distinct weight bytes each measured op cycles through (> 256 MB MALL)


def _copies(torch, arr, rows, cols):
    """The device (stream-layout) copy of the q4 matrix arr, cloned until the copies exceed
    ROTATE_BYTES."""
    import kq4
    t = kq4.prepare_dev(torch.from_numpy(arr.reshape(-1)).cuda(), rows, cols)
    n = max(2, int(ROTATE_BYTES // t.numel()) + 1)
    return [t] + [t.clone() for _ in range(n - 1)]


INT8_PEAK_TOPS = 5000.0


def roof_hbm(byts, us):
    a = byts / us / 1e3
    return {"bound": "hbm", "achieved": round(a, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(a / HBM_PEAK_GBS, 4)}


def roof_mfma(ops, us):
    a = ops / us / 1e6
    return {"bound": "mfma", "achieved": round(a, 1), "peak": INT8_PEAK_TOPS, "unit": "TOPS",
            "frac": round(a / INT8_PEAK_TOPS, 4)}


def run_extras(args):
    """The other BASELINE.json configs, each with its own roofline block (reported beside the
    headline line): config 1 (one 2B GEMV, M = 1), the 2B lm_head GEMV (M = 1), config 2 at
    M = 4 (the headline step),
    config 3 (Qwen3-8B decode GEMVs at M in {1,2,4,8}: us/call, GB/s against HBM peak, per op),
    config 4 (prefill GEMM at M in {512, 2048}: int8 TOPS against 5.0 POPS dense, per op) and
    config 5 (Qwen3-30B-A3B MoE FFN at T in {1, 64}), plus the Q8_0 weight form. Every measured
    op cycles through > 640 MB of distinct weight copies, so its weights stream from HBM; each
    is timed as a graph replay between HIP events on its stream (_time_graph)."""
    import torch

    import kq4

    out = {}
    # config 1: one q4 GEMV, M = 1, K = 2048 -> N = 6144 (the 2B FFN up-projection)
    rows1, cols1 = CFG["ffn"], CFG["hidden"]
    W1 = _copies(torch, synth.make_q4_weights(rows1, cols1, 11, **synth.SCALE_2B), rows1, cols1)
    x1 = torch.from_numpy(synth.make_activations(1, cols1, 7)).cuda()
    o1 = torch.empty((1, rows1), device="cuda")
    t1 = _time_graph(torch, lambda i, st: kq4.matmul_dev(o1, x1, W1[i], rows1, cols1, stream=st),
                     len(W1))
    b1 = rows1 * cols1 * 18 // 32 + cols1 * 4 + rows1 * 4
    out["config1_gemv_m1"] = {"us_per_call": round(t1, 3), "bytes": b1, "roofline": roof_hbm(b1, t1)}
    del W1
    # the 2B lm_head (vocab x hidden, 175 MB of q4 weights), one token on its M4f chain: the
    # largest decode GEMV of the model (vllm_safetensors.c:16844)
    rows_l = CFG["vocab"]
    WL = _copies(torch, synth.make_q4_weights(rows_l, cols1, 31, **synth.SCALE_2B), rows_l, cols1)
    ol = torch.empty((1, rows_l), device="cuda")
    tl = _time_graph(torch, lambda i, st: kq4.matmul_dev(ol, x1, WL[i], rows_l, cols1,
                                                        chain=kq4.CHAIN_GEMV32, stream=st),
                     len(WL))
    bl = rows_l * cols1 * 18 // 32 + cols1 * 4 + rows_l * 4
    out["lm_head_2b_m1"] = {"us_per_call": round(tl, 3), "bytes": bl, "roofline": roof_hbm(bl, tl)}
    del WL
    torch.cuda.empty_cache()
    # config 2 at M = 4: the headline step (28 layers' linear sets, one graph replay per step)
    g4 = run_gpu(argparse.Namespace(m=4, steps=max(10, args.steps // 2), warmup=args.warmup))
    out["config2_step_m4"] = {"ms_per_step": round(g4["ms_per_step"], 4),
                              "GBs": round(g4["value"], 1), "bytes_per_step": g4["total_bytes"],
                              "roofline": {"bound": "hbm", "achieved": round(g4["value"], 1),
                                           "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                           "frac": round(g4["value"] / HBM_PEAK_GBS, 4)},
                              "gate_up_us_per_call": round(g4["us_gate_up"], 3)}
    torch.cuda.empty_cache()
    cfg = synth.QWEN3_8B
    h, f = cfg["hidden"], cfg["ffn"]
    qkv = (cfg["q_heads"] + 2 * cfg["kv_heads"]) * cfg["head_dim"]
    G = _copies(torch, synth.make_q4_weights(f, h, 11, **synth.SCALE_8B), f, h)
    U = [g.clone() for g in G]
    D = _copies(torch, synth.make_q4_weights(h, f, 13, **synth.SCALE_8B), h, f)
    Q = _copies(torch, synth.make_q4_weights(qkv, h, 14, **synth.SCALE_8B), qkv, h)
    dec = {}
    for m in (1, 2, 4, 8):
        x = torch.from_numpy(synth.make_activations(m, h, 20 + m)).cuda()
        xf = torch.from_numpy(synth.make_activations(m, f, 30 + m)).cuda()
        og, ou = torch.empty((m, f), device="cuda"), torch.empty((m, f), device="cuda")
        od, oq = torch.empty((m, h), device="cuda"), torch.empty((m, qkv), device="cuda")
        t_gu = _time_graph(torch, lambda i, st: kq4.matmul_multi_dev(
            [og, ou], x, [G[i], U[i]], [f, f], h, stream=st), len(G))
        t_dn = _time_graph(torch, lambda i, st: kq4.matmul_dev(
            od, xf, D[i], h, f, stream=st), len(D))
        t_q = _time_graph(torch, lambda i, st: kq4.matmul_dev(
            oq, x, Q[i], qkv, h, stream=st), len(Q))
        # the FFN's second half: SiLU-multiply fused into the down projection, and the same as
        # two launches (the in-place product, then the down projection); |up| < 1 keeps the
        # repeatedly multiplied gate bounded
        xu = torch.rand((m, f), device="cuda") * 2 - 1
        xs = xf.clone()
        t_sd = _time_graph(torch, lambda i, st: kq4.matmul_silu_dev(
            od, xf, xu, D[i], h, f, stream=st), len(D))

        def unfused(i, st):
            kq4.silu_mul_dev(xs, xu, stream=st)
            kq4.matmul_dev(od, xs, D[i], h, f, stream=st)
        t_su = _time_graph(torch, unfused, len(D))
        # the attention block's input: RMSNorm + quantize in one pass feeding the QKV GEMV, and
        # the same as an RMSNorm launch followed by the QKV op
        nw = torch.rand(h, device="cuda") + 0.5
        xn = torch.empty_like(x)
        t_nq = _time_graph(torch, lambda i, st: kq4.rmsnorm_matmul_multi_dev(
            [oq], x, nw, 1e-6, [Q[i]], [qkv], h, stream=st), len(Q))

        def norm_then_qkv(i, st):
            kq4.rms_norm_dev(xn, x, nw, 1e-6, stream=st)
            kq4.matmul_dev(oq, xn, Q[i], qkv, h, stream=st)
        t_nu = _time_graph(torch, norm_then_qkv, len(Q))
        b_gu = 2 * f * h * 18 // 32 + m * h * 4 + 2 * m * f * 4
        b_dn = h * f * 18 // 32 + m * f * 4 + m * h * 4
        b_q = qkv * h * 18 // 32 + m * h * 4 + m * qkv * 4
        dec[f"M{m}"] = {
            "gate_up_us": round(t_gu, 2), "gate_up_GBs": round(b_gu / t_gu / 1e3, 1),
            "down_us": round(t_dn, 2), "down_GBs": round(b_dn / t_dn / 1e3, 1),
            "qkv_us": round(t_q, 2), "qkv_GBs": round(b_q / t_q / 1e3, 1),
            "silu_down_us": round(t_sd, 2),
            "silu_down_GBs": round((b_dn + m * f * 4) / t_sd / 1e3, 1),
            "silu_then_down_us": round(t_su, 2),
            "rmsnorm_qkv_us": round(t_nq, 2), "rmsnorm_then_qkv_us": round(t_nu, 2),
            "roofline_gate_up": roof_hbm(b_gu, t_gu), "roofline_down": roof_hbm(b_dn, t_dn),
            "roofline_qkv": roof_hbm(b_q, t_q)}
    out["qwen3_8b_decode"] = dec
    pre = {}
    for m in (512, 2048):
        x = torch.from_numpy(synth.make_activations(m, h, 40)).cuda()
        xf = torch.from_numpy(synth.make_activations(m, f, 41)).cuda()
        og = torch.empty((m, f), device="cuda")
        od = torch.empty((m, h), device="cuda")
        n = 4
        t_g = _time_graph(torch, lambda i, st: kq4.matmul_dev(
            og, x, G[i], f, h, stream=st), n, reps=2)
        t_d = _time_graph(torch, lambda i, st: kq4.matmul_dev(
            od, xf, D[i], h, f, stream=st), n, reps=2)
        ops = 2.0 * m * f * h
        pre[f"M{m}"] = {"gate_us": round(t_g, 1), "gate_TOPS": round(ops / t_g / 1e6, 1),
                        "down_us": round(t_d, 1), "down_TOPS": round(ops / t_d / 1e6, 1),
                        "roofline_gate": roof_mfma(ops, t_g), "roofline_down": roof_mfma(ops, t_d)}
    out["qwen3_8b_prefill"] = pre
    del G, U, D, Q
    torch.cuda.empty_cache()
    # the same shapes with Q8_0 weights (8x8 tiles), the reference's prefill format of dual VQF
    # files: prefill GEMM and the decode GEMV
    def q8_copies(rows, cols, seed):
        t = kq4.q8_prepare_dev(synth.make_q8_weights(rows, cols, seed), rows, cols)
        n = max(2, int(ROTATE_BYTES // t.numel()) + 1)
        return [t] + [t.clone() for _ in range(n - 1)]
    G8, D8 = q8_copies(f, h, 15), q8_copies(h, f, 16)
    q8 = {}
    for m in (1, 4, 512, 2048):
        x = torch.from_numpy(synth.make_activations(m, h, 70 + m)).cuda()
        xf = torch.from_numpy(synth.make_activations(m, f, 71 + m)).cuda()
        og = torch.empty((m, f), device="cuda")
        od = torch.empty((m, h), device="cuda")
        n, reps = (len(G8), 5) if m <= 8 else (4, 2)
        t_g = _time_graph(torch, lambda i, st: kq4.q8_matmul_dev(og, x, G8[i], f, h, stream=st),
                          n, reps=reps)
        t_d = _time_graph(torch, lambda i, st: kq4.q8_matmul_dev(od, xf, D8[i], h, f, stream=st),
                          n, reps=reps)
        if m <= 8:
            b_w = f * h * 34 // 32
            q8[f"M{m}"] = {"gate_us": round(t_g, 2),
                           "gate_GBs": round((b_w + m * h * 4 + m * f * 4) / t_g / 1e3, 1),
                           "down_us": round(t_d, 2),
                           "down_GBs": round((b_w + m * f * 4 + m * h * 4) / t_d / 1e3, 1)}
        else:
            ops = 2.0 * m * f * h
            q8[f"M{m}"] = {"gate_us": round(t_g, 1), "gate_TOPS": round(ops / t_g / 1e6, 1),
                           "down_us": round(t_d, 1), "down_TOPS": round(ops / t_d / 1e6, 1),
                           "gate_frac_int8_peak": round(ops / t_g / 1e6 / INT8_PEAK_TOPS, 4),
                           "down_frac_int8_peak": round(ops / t_d / 1e6 / INT8_PEAK_TOPS, 4)}
    out["qwen3_8b_q8_0"] = q8
    del G8, D8
    torch.cuda.empty_cache()
    mcfg = synth.QWEN3_30B_A3B_MOE
    d, ne, tk, ef = mcfg["hidden"], mcfg["experts"], mcfg["top_k"], mcfg["ef"]
    Gm, Um, Dm = synth.make_moe(mcfg, 50)
    layers = list(zip(_copies(torch, Gm, ne * ef, d), _copies(torch, Um, ne * ef, d),
                      _copies(torch, Dm, d, ne * ef)))
    moe = {}
    for T in (1, 64):
        X = torch.from_numpy(synth.make_activations(T, d, 60)).cuda()
        lg = torch.from_numpy(synth.make_logits(T, ne, 61)).cuda()
        sel = torch.empty((T, tk), dtype=torch.int32, device="cuda")
        pr = torch.empty((T, tk), device="cuda")
        Y = torch.empty((T, d), device="cuda")
        kq4.moe_route_dev(sel, pr, lg, tk)
        torch.cuda.synchronize()
        t = _time_graph(torch, lambda i, st: kq4.moe_ffn_dev(
            Y, X, sel, pr, *layers[i], ne, d, ef, stream=st), len(layers))
        n_exp = len(set(sel.cpu().numpy().reshape(-1).tolist()))
        byts = n_exp * 3 * ef * d * 18 // 32 + T * d * 8
        # the whole layer on the device: fp32 router logits (serial chains), top-k, expert FFN
        R = torch.randn((ne, d), device="cuda") * 0.02
        lgr = torch.empty((T, ne), device="cuda")
        t_lg = _time_graph(torch, lambda i, st: kq4.moe_router_logits_dev(lgr, R, X, stream=st),
                           len(layers))
        t_l = _time_graph(torch, lambda i, st: kq4.moe_layer_dev(
            Y, X, R, *layers[i], ne, tk, d, ef, stream=st), len(layers))
        moe[f"T{T}"] = {"us": round(t, 2), "experts": n_exp, "GBs": round(byts / t / 1e3, 1),
                        "roofline": roof_hbm(byts, t),
                        "router_logits_us": round(t_lg, 2), "layer_us": round(t_l, 2)}
    out["qwen3_30b_a3b_moe"] = moe
    return out


def cpu_baseline(m, budget_s=12.0):
    """The reference's own x86-64 code for every config (oracle/cpu_bench.py: seeded weights,
    median of >= 20 reps, all physical cores and the reference's nc - 2 default, MoE in both
    activation tracks). Without the reference build (oracle/_ref) it falls back to timing the
    oracle's scalar restatement of the headline step (kind "port", one thread, ~budget_s)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    if oracle.ref_available():
        import cpu_bench
        return cpu_bench.run(m)
    s = layer_mats()
    h, q, f = CFG["hidden"], s["q"][0], CFG["ffn"]
    w = {n: synth.make_q4_weights(r, c, 1 + i, **synth.SCALE_2B)
         for i, (n, (r, c)) in enumerate(s.items())}
    src = {"q": synth.make_activations(m, h, 7), "o": synth.make_activations(m, q, 8),
           "down": synth.make_activations(m, f, 9)}
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n == 0:
        for name, (rr, cc) in s.items():
            oracle.matmul(w[name], src.get(name, src["q"]), rr, cc)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return dict(value=round(step_bytes(m) / dt / 1e9, 3), unit="GB/s", cores=1, kind="port",
                sample=f"{n} layer linear sets (M={m}) through the oracle's scalar C, "
                       f"{dt * 1e3:.2f} ms per layer")


PROFILE_OPS = ("gemv_up_2b", "gemv_gate_up_2b", "gemv_gate_up_8b", "gemv_down_8b", "gemm_gate_8b",
               "gemm_down_8b", "moe_30b_a3b", "moe_layer_30b_a3b", "silu_down_8b",
               "rmsnorm_qkv_8b", "q8_gate_8b", "q8_down_8b", "gemv_8b_sweep")


def profile_gemv_sweep(reps):
    """The Qwen3-8B decode GEMVs as the extras time them - the fused gate/up pair and down, from
    fp32 activations, at M = 1, 2, 4, 8 - each launched `reps` times over rotating weight copies
    (> 640 MB, so the weights stream from HBM). In a kernel trace the GEMV's template arguments
    name M, and the grid (gate/up 768 row sets, down 128) names the op."""
    import torch

    import kq4

    kq4.init(0)
    st = torch.cuda.current_stream()
    cfg = synth.QWEN3_8B
    h, f = cfg["hidden"], cfg["ffn"]
    G = _copies(torch, synth.make_q4_weights(f, h, 11, **synth.SCALE_8B), f, h)
    U = [g.clone() for g in G]
    D = _copies(torch, synth.make_q4_weights(h, f, 13, **synth.SCALE_8B), h, f)
    for m in (1, 2, 4, 8):
        x = torch.from_numpy(synth.make_activations(m, h, 20 + m)).cuda()
        xf = torch.from_numpy(synth.make_activations(m, f, 30 + m)).cuda()
        og, ou = torch.empty((m, f), device="cuda"), torch.empty((m, f), device="cuda")
        od = torch.empty((m, h), device="cuda")
        for r in range(reps):
            kq4.matmul_multi_dev([og, ou], x, [G[r % len(G)], U[r % len(G)]], [f, f], h, stream=st)
        for r in range(reps):
            kq4.matmul_dev(od, xf, D[r % len(D)], h, f, stream=st)
        torch.cuda.synchronize()
    return dict(op="gemv_8b_sweep", reps=reps)


def profile_op(op, m, reps):
    """Launches one op `reps` times back to back (eager) for rocprofv3 runs: the 2B / 8B decode
    GEMVs, the 8B prefill GEMMs (m tokens), the Qwen3-30B-A3B MoE FFN or whole layer (router
    included; m tokens), the 8B SiLU-multiply + down and RMSNorm + QKV ops, or the 8B gate / down
    with Q8_0 weights (m tokens: GEMV up to 8, GEMM beyond). Launch i takes weight copy
    i % copies, the copies together over 640 MB (above the 256 MB Infinity Cache), so every
    launch streams its weights from HBM as in the timed extras."""
    import torch

    import kq4

    kq4.init(0)
    st = torch.cuda.current_stream()
    if op.startswith("moe"):
        cfg = synth.QWEN3_30B_A3B_MOE
        d, ne, tk, ef = cfg["hidden"], cfg["experts"], cfg["top_k"], cfg["ef"]
        G, U, D = synth.make_moe(cfg, 50)
        layers = list(zip(_copies(torch, G, ne * ef, d), _copies(torch, U, ne * ef, d),
                          _copies(torch, D, d, ne * ef)))
        X = torch.from_numpy(synth.make_activations(m, d, 60)).cuda()
        lg = torch.from_numpy(synth.make_logits(m, ne, 61)).cuda()
        sel = torch.empty((m, tk), dtype=torch.int32, device="cuda")
        pr = torch.empty((m, tk), device="cuda")
        Y = torch.empty((m, d), device="cuda")
        kq4.moe_route_dev(sel, pr, lg, tk, stream=st)
        R = torch.randn((ne, d), device="cuda") * 0.02
        for i in range(reps):
            Gd, Ud, Dd = layers[i % len(layers)]
            if op == "moe_layer_30b_a3b":
                kq4.moe_layer_dev(Y, X, R, Gd, Ud, Dd, ne, tk, d, ef, stream=st)
            else:
                kq4.moe_ffn_dev(Y, X, sel, pr, Gd, Ud, Dd, ne, d, ef, stream=st)
    elif op.startswith("q8"):
        h, f = synth.QWEN3_8B["hidden"], synth.QWEN3_8B["ffn"]
        rows, cols = (h, f) if "down" in op else (f, h)
        w = kq4.q8_prepare_dev(synth.make_q8_weights(rows, cols, 15), rows, cols)
        ws = [w] + [w.clone() for _ in range(max(1, int(ROTATE_BYTES // w.numel())))]
        x = torch.from_numpy(synth.make_activations(m, cols, 20)).cuda()
        out = torch.empty((m, rows), device="cuda")
        for i in range(reps):
            kq4.q8_matmul_dev(out, x, ws[i % len(ws)], rows, cols, stream=st)
    elif op in ("silu_down_8b", "rmsnorm_qkv_8b"):
        cfg = synth.QWEN3_8B
        h, f = cfg["hidden"], cfg["ffn"]
        if op == "silu_down_8b":
            ws = _copies(torch, synth.make_q4_weights(h, f, 13), h, f)
            g = torch.from_numpy(synth.make_activations(m, f, 21)).cuda()
            u = torch.rand((m, f), device="cuda") * 2 - 1
            out = torch.empty((m, h), device="cuda")
            for i in range(reps):
                kq4.matmul_silu_dev(out, g, u, ws[i % len(ws)], h, f, stream=st)
        else:
            qkv = (cfg["q_heads"] + 2 * cfg["kv_heads"]) * cfg["head_dim"]
            ws = _copies(torch, synth.make_q4_weights(qkv, h, 14), qkv, h)
            x = torch.from_numpy(synth.make_activations(m, h, 22)).cuda()
            nw = torch.rand(h, device="cuda") + 0.5
            out = torch.empty((m, qkv), device="cuda")
            for i in range(reps):
                kq4.rmsnorm_matmul_multi_dev([out], x, nw, 1e-6, [ws[i % len(ws)]], [qkv], h,
                                             stream=st)
    else:
        cfg = CFG if op.endswith("2b") else synth.QWEN3_8B
        h, f = cfg["hidden"], cfg["ffn"]
        rows, cols = (h, f) if "down" in op else (f, h)
        nmat = 2 if "gate_up" in op else 1
        mats = [_copies(torch, synth.make_q4_weights(rows, cols, 11 + i), rows, cols)
                for i in range(nmat)]
        x = torch.from_numpy(synth.make_activations(m, cols, 20)).cuda()
        outs = [torch.empty((m, rows), device="cuda") for _ in range(nmat)]
        for i in range(reps):
            kq4.matmul_multi_dev(outs, x, [c[i % len(c)] for c in mats], [rows] * nmat, cols,
                                 stream=st)
    torch.cuda.synchronize()
    return dict(op=op, m=m, reps=reps)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--m", type=int, default=1, help="tokens per step (decode batch)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the config 3-5 sub-results (8B decode, prefill GEMM, MoE)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 512 MiB device copy (PMC byte-counter calibration)")
    ap.add_argument("--profile-op", choices=PROFILE_OPS,
                    help="only launch this op --reps times (for rocprofv3 runs); --m = tokens")
    ap.add_argument("--reps", type=int, default=5)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard along weight rows for the dense matmuls and along experts "
              "for the MoE, each GPU running these kernels on its share)",
              file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        print(json.dumps(copy_calibration()))
        return
    if args.profile_op == "gemv_8b_sweep":
        print(json.dumps(profile_gemv_sweep(args.reps)))
        return
    if args.profile_op:
        print(json.dumps(profile_op(args.profile_op, args.m, args.reps)))
        return
    g = run_gpu(args)
    traffic, traffic_commit = profiled_traffic(args.m)
    line = {
        "metric": METRIC,
        "value": round(g["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_per_step"], 4),
        "eager": {"ms_per_step": round(g["ms_eager"], 4), "value": round(g["value_eager"], 2)},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"qwen3-vl-2b decode-step linear set (QKV, O+res, gate/up, "
                               f"down+res) x {CFG['layers']} layers, M={args.m}",
                   "global_batch": args.m, "bytes_per_step": g["total_bytes"],
                   "launch": "one HIP graph replay per step (4 launches per layer)",
                   "weights": "q4_0 4x4 tiles (repacked once into the kq4 stream layout), "
                              "int8 block-32 activations"},
        "gate_up_us_per_call": round(g["us_gate_up"], 3),
        "roofline": {"bound": "hbm", "achieved": round(g["achieved"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(g["achieved"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "traffic_measured_at_commit": traffic_commit,
                     "kernel": "kq4_gemv_kernel (fused gate/up, 2 x 6144x2048)"},
    }
    if not args.no_extras:
        line["extras"] = run_extras(args)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.m, args.cpu_seconds)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
