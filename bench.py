#!/usr/bin/env python3
"""Benchmark: one Qwen3.5-4B-shaped decode step over the compute cores of 32
hybrid layers at context 8192, on one MI355X.

Per step (models/llm/qwen3_5.cpp:1278-1356 with the projections left out):
  * 8 full-attention cores (layers 3, 7, ..., 31): q/k RMSNorm, partial RoPE,
    fp16 KV append, GQA attention over 8192 keys (16 q / 4 kv heads, D 256),
    sigmoid output gate;
  * 24 Gated-DeltaNet cores (16 key / 32 value heads x 128, fp32 state) with
    the gated-RMSNorm epilogue;
  * 32 LUT6 SwiGLU FFN blocks 2560 -> 9216 -> 2560 with RMSNorm and residual.
Inputs are synthetic (seeded), resident in HBM before timing; the step runs as
one persistent-kernel launch (falls back to a HIP-graph replay of the eager
launch sequence where the persistent step does not fit).  Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))

METRIC = "µs per decode step (attn+DeltaNet+LUT6, 4B shape); HBM GB/s as % of peak"
HBM_PEAK_GBPS = 8000.0
MODE_NAMES = {0: "eager launches", 1: "hip graph replay", 6: "persistent kernel, one launch per step"}
# HBM bytes per launch of the step kernel from two rocprofv3 --pmc runs
# (FETCH_SIZE, WRITE_SIZE; KiB per dispatch), each scaled by what the counter
# reads for a 1 GiB device copy in the same run (fetch 524338 KiB -> factor
# 1.99981; write 1048576 KiB -> factor 1.0): fetch 1040983 KiB, write 62939 KiB.
TRAFFIC = {"step_kernel": 2196179422}

CFG = dict(hidden=2560, inter=9216, layers=32, n_heads=16, n_kv_heads=4, head_dim=256, rot_dim=64,
           theta=1e7, eps=1e-6, lin_k_heads=16, lin_v_heads=32, lin_dim=128, ctx=8192)


def step_bytes(c=CFG):
    """Algorithmic HBM bytes per step: every input read once, every output
    written once (KV as fp16, DeltaNet state fp32 read + write, LUT6 at 0.75
    B/weight plus the fp16 LUTs)."""
    n_attn = c["layers"] // 4
    n_dn = c["layers"] - n_attn
    H, I, D = c["hidden"], c["inter"], c["head_dim"]
    kv = n_attn * c["ctx"] * c["n_kv_heads"] * D * 2 * 2
    attn_io = n_attn * (c["n_heads"] * 2 * D * 4 + 2 * c["n_kv_heads"] * D * 4 + 2 * D * 4
                        + c["n_heads"] * D * 4)
    state = n_dn * c["lin_v_heads"] * c["lin_dim"] ** 2 * 4 * 2
    dn_io = n_dn * (2 * c["lin_k_heads"] * 128 * 4 + 3 * c["lin_v_heads"] * 128 * 4
                    + 4 * c["lin_v_heads"] * 4 + 128 * 4)
    w = c["layers"] * (3 * H * I * 3 // 4 + (2 * I // 32 + H // 32) * 64 * 2)
    ffn_io = c["layers"] * (2 * H * 4 + H * 4 + I * 4 * 2)
    return dict(kv=kv, state=state, lut6=w, io=attn_io + dn_io + ffn_io,
                total=kv + state + w + attn_io + dn_io + ffn_io)


def gateup_bytes(c=CFG):
    """Algorithmic bytes of one gate/up launch: two LUT6 matrices [inter][hidden],
    their LUTs, x and the norm weight read once, g and u written once."""
    H, I = c["hidden"], c["inter"]
    return 2 * (I * H * 3 // 4 + (I // 32) * 64 * 2) + 2 * H * 4 + 2 * I * 4


def build_step(anelm, torch, dev, seed=0, mode=None):
    """Allocates the synthetic 4B-shaped model state and returns (step, keep, x)."""
    c = CFG
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    H, I, D = c["hidden"], c["inter"], c["head_dim"]
    Hq, Hkv, Hk, Hv, dl = c["n_heads"], c["n_kv_heads"], c["lin_k_heads"], c["lin_v_heads"], c["lin_dim"]
    ctx = c["ctx"]

    def randn(*shape, std=1.0, dtype=torch.float32):
        return (torch.randn(*shape, generator=g, device=dev) * std).to(dtype)

    def randbytes(*shape):
        return torch.randint(0, 256, shape, generator=g, device=dev, dtype=torch.uint8)

    def lut(rows):
        return randn(rows // 32, 64, std=0.02, dtype=torch.float16)

    keep = []
    layers = (anelm.HybridLayer * c["layers"])()
    for i in range(c["layers"]):
        L = layers[i]
        t = {}
        if (i + 1) % 4 == 0:
            L.kind = anelm.LAYER_ATTENTION
            t["q_gate"] = randn(Hq, 2 * D)
            t["k"] = randn(Hkv, D)
            t["v"] = randn(Hkv, D)
            t["k_cache"] = randn(ctx, Hkv, D, dtype=torch.float16)
            t["v_cache"] = randn(ctx, Hkv, D, dtype=torch.float16)
            t["q_norm_w"] = 1 + randn(D, std=0.02)
            t["k_norm_w"] = 1 + randn(D, std=0.02)
            t["core_out"] = torch.empty(Hq * D, device=dev)
            L.cache_start, L.cache_len, L.cache_capacity, L.pos = 0, ctx - 1, ctx, ctx - 1
        else:
            L.kind = anelm.LAYER_DELTANET
            t["state"] = randn(Hv, dl, dl, std=0.1)
            t["dn_q"] = randn(Hk, dl)
            t["dn_k"] = randn(Hk, dl)
            t["dn_v"] = randn(Hv, dl)
            t["dn_a"] = randn(Hv)
            t["dn_b"] = randn(Hv)
            t["dn_A"] = torch.exp(torch.rand(Hv, generator=g, device=dev) * 2.772588722239781)
            t["dn_dt_bias"] = randn(Hv)
            t["dn_z"] = randn(Hv, dl)
            t["dn_norm_w"] = 1 + randn(dl, std=0.02)
            t["core_out"] = torch.empty(Hv * dl, device=dev)
            L.dn_flags = 1 | 4
        t["ffn_norm_w"] = 1 + randn(H, std=0.02)
        t["gate_w"] = randbytes(I, H * 3 // 4)
        t["gate_lut"] = lut(I)
        t["up_w"] = randbytes(I, H * 3 // 4)
        t["up_lut"] = lut(I)
        t["down_w"] = randbytes(H, I * 3 // 4)
        t["down_lut"] = lut(H)
        for name, ten in t.items():
            setattr(L, name, ten.data_ptr())
        keep.append(t)
    x = randn(H)
    h = torch.empty(2 * I, device=dev)
    keep.append({"x": x, "h": h})
    dims = anelm.HybridDims(H, I, Hq, Hkv, D, c["rot_dim"], 0, c["theta"], c["eps"], Hk, Hv, dl)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    modes = [mode] if mode is not None else [anelm.STEP_PERSISTENT | anelm.STEP_STATIC, anelm.STEP_GRAPH]
    for md in modes:
        handle = ctypes.c_void_p()
        rc = anelm.status("anelm_hybrid_step_create", ctypes.byref(handle), ctypes.byref(dims), layers,
                          c["layers"], ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(h.data_ptr()), md,
                          ctypes.c_void_p(stream.cuda_stream))
        if rc == 0:
            break
        print(f"step mode {md} unavailable: {anelm.last_error()}", file=sys.stderr)
    else:
        raise RuntimeError("no decode-step mode could be created")
    keep.append((layers, dims))
    return handle, keep, x, md


def time_gateup(anelm, torch, keep, n=50):
    """Average duration of the LUT6 gate/up kernel (the step's largest launch),
    timed with HIP events on the stream it is launched on."""
    c = CFG
    xv = torch.randn(c["hidden"], device="cuda")
    gv = torch.empty(c["inter"], device="cuda")
    uv = torch.empty(c["inter"], device="cuda")
    stream = torch.cuda.current_stream()
    s = ctypes.c_void_p(stream.cuda_stream)
    # rotate over all 32 layers' weights so every launch streams from HBM
    mats = [k for k in keep if isinstance(k, dict) and "gate_w" in k]
    arglist = []
    for m in mats:
        arglist.append((ctypes.c_void_p(gv.data_ptr()), ctypes.c_void_p(uv.data_ptr()),
                        ctypes.c_void_p(xv.data_ptr()),
                        ctypes.c_void_p(m["ffn_norm_w"].data_ptr()), ctypes.c_float(c["eps"]),
                        ctypes.c_void_p(m["gate_w"].data_ptr()), ctypes.c_void_p(m["gate_lut"].data_ptr()),
                        ctypes.c_void_p(m["up_w"].data_ptr()), ctypes.c_void_p(m["up_lut"].data_ptr()),
                        c["hidden"], c["inter"], s))
    for a in arglist[:4]:
        anelm.call("anelm_lut6_gate_up", *a)
    durs = []
    for i in range(n):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        anelm.call("anelm_lut6_gate_up", *arglist[i % len(arglist)])
        e1.record(stream)
        durs.append((e0, e1))
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in durs]
    return statistics.mean(ms) * 1e3, statistics.median(ms) * 1e3


def cpu_baseline(seconds=12.0):
    """The oracle (a single-threaded C restatement of the reference cpu_ops
    path) on a bounded sample of the same step: one block of four layers
    (1 attention over an fp32 8192-key cache as the reference stores it,
    3 DeltaNet, 4 LUT6 FFN blocks evaluated as dequantise + fp32 matvec),
    repeated for about `seconds`, scaled x8 to the 32-layer step."""
    import numpy as np
    from workloads import load_oracle
    orc = load_oracle()
    c = CFG
    rng = np.random.default_rng(7)
    H, I, D, ctx = c["hidden"], c["inter"], c["head_dim"], c["ctx"]
    Hq, Hkv = c["n_heads"], c["n_kv_heads"]
    kc = rng.standard_normal((ctx, Hkv, D), dtype=np.float32)
    vc = rng.standard_normal((ctx, Hkv, D), dtype=np.float32)
    qg = rng.standard_normal((Hq, 2 * D), dtype=np.float32)
    kn = rng.standard_normal((Hkv, D), dtype=np.float32)
    w = np.ones(D, np.float32)
    state = (0.1 * rng.standard_normal((32, 128, 128))).astype(np.float32)
    dq = rng.standard_normal((16, 128), dtype=np.float32)
    dv = rng.standard_normal((32, 128), dtype=np.float32)
    dab = rng.standard_normal(32).astype(np.float32)
    ffn = [(rng.integers(0, 256, (I, H * 3 // 4), dtype=np.uint8),
            rng.integers(0, 256, (I, H * 3 // 4), dtype=np.uint8),
            rng.integers(0, 256, (H, I * 3 // 4), dtype=np.uint8)) for _ in range(4)]
    lut_i = (0.02 * rng.standard_normal((I // 32, 64))).astype(np.float16).view(np.uint16)
    lut_h = (0.02 * rng.standard_normal((H // 32, 64))).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(H).astype(np.float32)

    def block():
        # attention core, as qwen3_5.cpp:944-1002 runs it on an fp32 ring cache
        q = orc.rmsnorm(qg.reshape(Hq, 2, D)[:, 0], w)
        k = orc.rmsnorm(kn, w)
        q, k = orc.apply_rope(q, k, Hq, Hkv, D, D, D, c["rot_dim"], ctx - 1, c["theta"])
        kc[ctx - 1] = k
        out = orc.gqa_attention(q, kc, vc, Hq, Hkv, D, D, 0, ctx, ctx)
        orc.mul_sigmoid(out, qg.reshape(Hq, 2, D)[:, 1])
        for _ in range(3):
            orc.deltanet_decode(state, dq, dq, dv, dab, dab, np.abs(dab), dab, 5,
                                dv, np.ones(128, np.float32))
        for g_, u_, d_ in ffn:
            orc.lut6_ffn(x, (g_, lut_i), (u_, lut_i), (d_, lut_h), H, I)

    block()
    reps = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(reps) < 2:
        t0 = time.perf_counter()
        block()
        reps.append(time.perf_counter() - t0)
    per_step_us = statistics.median(reps) * 8 * 1e6
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(per_step_us, 1), "unit": "us/step", "cores": 1, "kind": "port",
            "sample": f"{len(reps)} runs of one 4-layer block (1 attention over 8192 fp32 keys, "
                      f"3 DeltaNet, 4 LUT6 FFN as dequant+matvec), median x8 layers-blocks; "
                      f"oracle/anelm_oracle.c, 1 thread, {cpu_model}, nproc {os.cpu_count()}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--mode", choices=["persistent", "graph", "eager"], default=None,
                    help="decode-step execution (default: persistent, else graph)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                    help="after the timed steps, copy MB MiB device-to-device once (a kernel of known "
                         "traffic that scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this benchmark measures one GPU; the decode step does not "
                                   "shard across GPUs in this build (run with --gpus 1)"}))
        sys.exit(2)

    import torch
    from workloads import load_package
    anelm = load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        md = {"persistent": anelm.STEP_PERSISTENT | anelm.STEP_STATIC, "graph": anelm.STEP_GRAPH,
              "eager": anelm.STEP_EAGER, None: None}[args.mode]
        handle, keep, x, mode = build_step(anelm, torch, dev, mode=md)
        s = ctypes.c_void_p(stream.cuda_stream)
        for _ in range(args.warmup):
            anelm.call("anelm_hybrid_step_run", handle, s)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(args.steps):
            anelm.call("anelm_hybrid_step_run", handle, s)
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms_total = e0.elapsed_time(e1)
        us_step = ms_total * 1e3 / args.steps
        assert torch.isfinite(x).all(), "non-finite hidden state"
        st = ctypes.c_int(0)
        anelm.call("anelm_hybrid_step_status", handle, ctypes.byref(st))
        assert st.value == 0, "a grid barrier of the persistent step timed out"
        gu_avg, gu_med = time_gateup(anelm, torch, keep)
        anelm.call("anelm_hybrid_step_destroy", handle)
        if args.copy_probe:
            src = torch.empty(args.copy_probe << 18, device=dev)
            dst = torch.empty_like(src)
            torch.cuda.synchronize()
            dst.copy_(src)
            torch.cuda.synchronize()
            del src, dst
        persistent = bool(mode & anelm.STEP_PERSISTENT)

    b = step_bytes()
    gbps = b["total"] / (us_step * 1e-6) / 1e9
    gu_b = gateup_bytes()
    gu_gbps = gu_b / (gu_avg * 1e-6) / 1e9
    result = {
        "metric": METRIC,
        "value": round(us_step, 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random-init weights, fp16 KV, LUT6 indices)",
        "config": {"workload": "qwen3.5-4b decode step over the compute cores of 32 hybrid layers: "
                               "8 full-attention (16q/4kv, D256, partial RoPE 64, ctx 8192 fp16 KV), "
                               "24 Gated-DeltaNet (16k/32v heads x128, fp32 state, gated norm), "
                               "32 LUT6 SwiGLU FFN 2560->9216->2560",
                   "batch": 1, "context": CFG["ctx"], "layers": CFG["layers"],
                   "execution": MODE_NAMES.get(mode, str(mode))},
        "hbm_GBps": round(gbps, 1),
        "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
        "algorithmic_bytes_per_step": b["total"],
        "wall_s": round(wall, 4),
    }
    if persistent:
        # one kernel per step: its launch duration is the step time (HIP events
        # on the stream it runs on), its algorithmic bytes are the step's
        result["roofline"] = {"bound": "hbm", "kernel": "step_kernel (whole 32-layer decode step)",
                              "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                              "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": TRAFFIC.get("step_kernel"),
                              "bytes_per_launch": b["total"], "avg_us": round(us_step, 3)}
    else:
        result["roofline"] = {"bound": "hbm", "kernel": "lut6_tile_kernel (gate+up, 2 x 9216x2560)",
                              "achieved": round(gu_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                              "frac": round(gu_gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                              "bytes_per_launch": gu_b, "avg_us": round(gu_avg, 3)}
    result["lut6_gate_up"] = {"avg_us": round(gu_avg, 3), "median_us": round(gu_med, 3),
                              "GBps": round(gu_gbps, 1), "bytes_per_launch": gu_b}
    if not args.skip_cpu:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
