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
import math
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
# HBM bytes per launch of the step kernel from rocprofv3 --pmc runs of this
# script: fetched = 32 x TCC_EA0_RDREQ_32B + 64 x TCC_EA0_RDREQ_64B + 128 x
# TCC_EA0_RDREQ_128B (summed over the L2 channels) = 2,139,283,283 B; written =
# WRITE_SIZE x 1024 = 71,560,499 B.  The same counters read 1,073,768,640 B
# fetched and 1,073,741,824 B written for a 1 GiB device copy in the same runs.
TRAFFIC = {"step_kernel": 2210843782}

CFG = dict(hidden=2560, inter=9216, layers=32, n_heads=16, n_kv_heads=4, head_dim=256, rot_dim=64,
           theta=1e7, eps=1e-6, lin_k_heads=16, lin_v_heads=32, lin_dim=128, ctx=8192)
# the reference's default model (models/llm/qwen3_5.h:51-69)
CFG_08B = dict(hidden=1024, inter=3584, layers=24, n_heads=8, n_kv_heads=2, head_dim=256, rot_dim=64,
               theta=1e7, eps=1e-6, lin_k_heads=16, lin_v_heads=16, lin_dim=128, ctx=8192)


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


def proj_bytes(c=CFG):
    """Algorithmic bytes the projections around the cores add to a step: the
    LUT6 first projections (DeltaNet 2560 -> 12352: qkv | z | a | b;
    attention 2560 -> 10240: q_gate | k | v), o_proj 4096 -> 2560, their LUTs,
    the input norm weights and the DeltaNet conv rings (read + write) and
    conv weights."""
    n_attn = c["layers"] // 4
    n_dn = c["layers"] - n_attn
    H = c["hidden"]
    f_dn = 2 * c["lin_k_heads"] * 128 + 2 * c["lin_v_heads"] * 128 + 2 * c["lin_v_heads"]
    f_at = c["n_heads"] * 2 * c["head_dim"] + 2 * c["n_kv_heads"] * c["head_dim"]
    o_in = c["n_heads"] * c["head_dim"]
    qkv = 2 * c["lin_k_heads"] * 128 + c["lin_v_heads"] * 128

    def lut6(out, inp):
        return out * inp * 3 // 4 + (out // 32) * 128

    w = n_dn * lut6(f_dn, H) + n_attn * lut6(f_at, H) + c["layers"] * (lut6(H, o_in) + H * 4)
    conv = n_dn * qkv * (3 * 4 * 2 + 4 * 4)
    return w + conv


def build_step(anelm, torch, dev, seed=0, mode=None, proj=False, c=CFG):
    """Allocates the synthetic model state of shape c (the 4B shape by
    default) and returns (step, keep, x).  With proj, every layer also carries
    its projections (input norm + first projection, DeltaNet conv ring,
    o_proj) and the step runs whole layers."""
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
        if proj:
            attn = (i + 1) % 4 == 0
            f_out = Hq * 2 * D + 2 * Hkv * D if attn else 2 * Hk * dl + 2 * Hv * dl + 2 * Hv
            t["in_norm_w"] = 1 + randn(H, std=0.02)
            t["first_w"] = randbytes(f_out, H * 3 // 4)
            t["first_lut"] = lut(f_out)
            t["o_w"] = randbytes(H, (Hq * D if attn else Hv * dl) * 3 // 4)
            t["o_lut"] = lut(H)
            t["proj"] = torch.empty(f_out, device=dev)
            if not attn:
                qkv = 2 * Hk * dl + Hv * dl
                t["conv_state"] = randn(qkv, 3, std=0.5)
                t["conv_w"] = randn(qkv, 4, std=0.5)
        for name, ten in t.items():
            setattr(L, name, ten.data_ptr())
        keep.append(t)
    x = randn(H)
    h = torch.empty(2 * I, device=dev)
    keep.append({"x": x, "h": h})
    dims = anelm.HybridDims(H, I, Hq, Hkv, D, c["rot_dim"], 0, c["theta"], c["eps"], Hk, Hv, dl, 4)
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


MFMA_F16_PEAK_TFLOPS = 2500.0   # MI355X dense fp16 MFMA, published


def _gpu_us(torch, fn, reps, warm=2):
    """Average GPU time of fn() on the current stream, HIP events around `reps`
    calls queued behind a GPU-side sleep, so host launch gaps are not timed."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(2.0e9 * 40e-6 * reps))
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def _hbm(us, nbytes):
    gbps = nbytes / (us * 1e-6) / 1e9
    return {"us": round(us, 3), "bytes": int(nbytes), "GBps": round(gbps, 1),
            "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4)}


def measure_cores(anelm, torch, dev, seed=11):
    """The other workloads of the path, each timed alone on one GPU with its
    roofline: decode attention (0.8B shape), DeltaNet decode, causal prefill
    attention and chunked DeltaNet prefill at 4096 tokens, and the pieces of the
    32-sequence batched decode (paged attention, batched DeltaNet, LUT6 LM head
    top-32)."""
    import numpy as np
    from workloads import attn_decode_case
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def randn(*shape, std=1.0, dtype=torch.float32):
        return (torch.randn(*shape, generator=g, device=dev) * std).to(dtype)

    def l2n(t):
        return t / t.norm(dim=-1, keepdim=True)

    res = {}
    # decode attention, 8 q / 2 kv heads, D 256, 512 cached keys + the new one
    c = attn_decode_case(seed)
    cap = 1024
    kc = torch.zeros(cap, 2, 256, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    kc[:c.length].copy_(torch.from_numpy(c.k_cache[:c.length].view(np.float16)))
    vc[:c.length].copy_(torch.from_numpy(c.v_cache[:c.length].view(np.float16)))
    qg, k1, v1 = (torch.from_numpy(a).to(dev) for a in (c.q_gate, c.k, c.v))
    qn, kn = torch.from_numpy(c.q_norm_w).to(dev), torch.from_numpy(c.k_norm_w).to(dev)
    out = torch.empty(8, 256, device=dev)

    def c1():
        anelm.ops.full_attn_decode(qg, k1, v1, kc, vc, qn, kn, anelm.ops.KVRing(cap, 0, c.length), 8, 2, 256,
                                   64, c.length, out=out)
    res["decode_attention_0.8b"] = dict(_hbm(_gpu_us(torch, c1, 200), 1079296), keys=c.length + 1)

    # DeltaNet decode, 16 heads x 128 x 128 fp32 state
    H = 16
    st = randn(H, 128, 128, std=0.1)
    dq, dk = l2n(randn(H, 128)), l2n(randn(H, 128))
    dv = randn(H, 128)
    da, db, ddt = randn(H), randn(H), randn(H)
    dA = torch.exp(torch.rand(H, generator=g, device=dev) * math.log(16.0))
    y = torch.empty(H, 128, device=dev)

    def c2():
        anelm.ops.deltanet_decode(st, dq, dk, dv, da, db, dA, ddt, 0, out=y)
    res["deltanet_decode"] = _hbm(_gpu_us(torch, c2, 200), 2129920)

    # causal prefill attention, S 4096, 16 q / 4 kv heads, D 256
    S = 4096
    q = randn(S, 16, 256, dtype=torch.float16)
    k = randn(S, 4, 256, dtype=torch.float16)
    v = randn(S, 4, 256, dtype=torch.float16)
    us = _gpu_us(torch, lambda: anelm.ops.attn_prefill(q, k, v), 20)
    flops = 4 * 256 * 16 * S * (S + 1) // 2
    tf = flops / (us * 1e-6) / 1e12
    res["prefill_attention_4096"] = {"us": round(us, 2), "flops": flops, "TFLOPs": round(tf, 1),
                                     "frac_mfma": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
    del q, k, v

    # chunked DeltaNet prefill, S 4096, 16 key / 32 value heads, chunk 64
    Hk, Hv = 16, 32
    st = randn(Hv, 128, 128, std=0.1)
    pq, pk = l2n(randn(S, Hk, 128)), l2n(randn(S, Hk, 128))
    pv = randn(S, Hv, 128)
    pa, pb = randn(S, Hv), randn(S, Hv)
    pdt = randn(Hv)
    pA = torch.exp(torch.rand(Hv, generator=g, device=dev) * math.log(16.0))
    us = _gpu_us(torch, lambda: anelm.ops.deltanet_prefill(st, pq, pk, pv, pa, pb, pA, pdt, 1), 10)
    r = _hbm(us, 206569472)
    r["GFLOPs_recurrent_form"] = round(15.03e9 / (us * 1e-6) / 1e9, 1)
    res["deltanet_prefill_4096"] = r
    del pq, pk, pv, pa, pb

    # prompt prefill through the layer cores over their state, 4096 tokens
    # (generate.cpp:55-85 runs the decode core once per prompt token): full
    # attention from the first projection's q_gate / k / v (q/k RMSNorm, RoPE
    # at each position, fp16 append into an empty 8192-key ring, the causal
    # MFMA core, the sigmoid gate) ...
    qg = randn(S, 16, 512)
    kx, vx = randn(S, 4, 256), randn(S, 4, 256)
    qnw, knw = 1 + randn(256, std=0.02), 1 + randn(256, std=0.02)
    kc = torch.zeros(8192, 4, 256, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    tab = anelm.ops.rope_table(64, S, 1e7, dev)
    ring = anelm.ops.KVRing(8192)

    def attn_layer():
        ring.start.value, ring.len.value = 0, 0
        anelm.ops.full_attn_prefill(qg, kx, vx, kc, vc, qnw, knw, ring, 16, 4, 256, 64, 0, rope_table=tab,
                                    rope_rows=S)
    us = _gpu_us(torch, attn_layer, 10)
    tf = flops / (us * 1e-6) / 1e12
    res["prompt_prefill_attention_layer_4096"] = {
        "us": round(us, 2), "TFLOPs": round(tf, 1), "frac_mfma": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
        "composition": "q/k RMSNorm, RoPE per position, fp16 ring append, causal MFMA core, sigmoid gate"}
    del qg, kx, vx, kc, vc
    # ... and Gated DeltaNet from its projection rows (conv ring + SiLU over
    # the prompt, l2 norm, gates, the chunked recurrence, rmsnorm_gated)
    qkv = 2 * Hk * 128 + Hv * 128
    proj = randn(S, qkv + Hv * 128 + 2 * Hv)
    conv_w, conv_st = randn(qkv, 4, std=0.5), randn(qkv, 3, std=0.5)
    nw = 1 + randn(128, std=0.02)
    st = randn(Hv, 128, 128, std=0.1)
    pos = ctypes.c_int(0)

    def dn_layer():
        pos.value = 0
        anelm.ops.deltanet_prefill_from_proj(st, conv_st, pos, proj, conv_w, pA, pdt, nw, Hk, 1 | 4)
    us = _gpu_us(torch, dn_layer, 10)
    res["prompt_prefill_deltanet_layer_4096"] = {
        "us": round(us, 2),
        "composition": "conv1d ring + SiLU, l2 norm, gates, chunked recurrence, rmsnorm_gated with z"}
    del proj, st

    # 32-sequence batched decode, per layer: paged attention over ragged
    # lengths U[256, 16384] (16-token pages, shuffled page table) ...
    rng = np.random.default_rng(seed)
    n_seq, P = 32, 16
    lens = rng.integers(256, 16385, n_seq).astype(np.int32)
    npg = (lens + P - 1) // P
    n_pages = int(npg.sum())
    perm = rng.permutation(n_pages).astype(np.int32)
    table = np.zeros((n_seq, int(npg.max())), np.int32)
    off = 0
    for s in range(n_seq):
        table[s, :npg[s]] = perm[off:off + npg[s]]
        off += npg[s]
    kp = randn(n_pages, 4, P, 256, dtype=torch.float16)
    vp = randn(n_pages, 4, P, 256, dtype=torch.float16)
    qg = randn(n_seq, 16, 512)
    kb, vb = randn(n_seq, 4, 256), randn(n_seq, 4, 256)
    qnw, knw = 1 + randn(256, std=0.02), 1 + randn(256, std=0.02)
    tb = torch.from_numpy(table).to(dev)
    lb = torch.from_numpy(lens - 1).to(dev)          # cached keys; the step appends the last one
    ob = torch.empty(n_seq, 16, 256, device=dev)
    rope = anelm.ops.rope_table(64, 16385, 1e7, dev)
    us = _gpu_us(torch, lambda: anelm.ops.attn_decode_paged_step(
        qg, kb, vb, kp, vp, tb, lb, qnw, knw, int(lens.max()), 16, 4, 256, P, 64, rope_tab=rope, out=ob), 10)
    r = _hbm(us, int(lens.sum()) * 4 * 256 * 2 * 2)
    r["sum_len"] = int(lens.sum())
    r["composition"] = "q/k RMSNorm, RoPE, fp16 page append, attention, gate per sequence"
    res["batch32_paged_attention_layer"] = r
    del kp, vp
    # ... DeltaNet decode of all 32 sequences in one launch (1024 value heads,
    # the layer's A / dt_bias / norm weight shared, gated norm) ...
    Hk, Hv = 16 * n_seq, 32 * n_seq
    st = randn(Hv, 128, 128, std=0.1)
    bq, bk = l2n(randn(Hk, 128)), l2n(randn(Hk, 128))
    bv, bz = randn(Hv, 128), randn(Hv, 128)
    ba, bb, bdt = randn(Hv), randn(Hv), randn(32)
    bA = torch.exp(torch.rand(32, generator=g, device=dev) * math.log(16.0))
    bnw = 1 + randn(128, std=0.02)
    by = torch.empty(Hv, 128, device=dev)
    us = _gpu_us(torch, lambda: anelm.ops.deltanet_decode_batched(st, bq, bk, bv, ba, bb, bA, bdt, 1 | 4, bz, bnw,
                                                                  n_seq, out=by), 20)
    res["batch32_deltanet_layer"] = _hbm(us, Hv * 128 * 128 * 4 * 2 + (2 * Hk + 3 * Hv) * 128 * 4)
    del st
    # ... and the LM head: top-32 of a [262144][2560] LUT6 matrix for 32 fp16-valued inputs
    V, D = 262144, 2560
    w = torch.randint(0, 256, (V, D * 3 // 4), generator=g, device=dev, dtype=torch.uint8)
    lut = randn(V // 32, 64, std=0.02, dtype=torch.float16)
    hx = randn(n_seq, D, dtype=torch.float16).float()
    us = _gpu_us(torch, lambda: anelm.ops.lut6_topk(w, lut, hx, V, D, 32), 10)
    res["batch32_lm_head_top32"] = _hbm(us, V * D * 3 // 4 + (V // 32) * 128 + n_seq * D * 4)
    return res


def measure_batch32_step(anelm, torch, dev, seed=12, reps=5):
    """32 concurrent sequences at the 4B shape through one decode step of 32
    hybrid layers with the batched-step executor (anelm_batch_step): per
    full-attention layer the fused step of every sequence over its own
    shuffled 16-token pages (q/k RMSNorm, RoPE at the sequence's position,
    fp16 page append, attention over its ragged U[256, 16384] keys, gate);
    per DeltaNet layer one launch over the 32 x 32 value heads (own fp32
    state each, gated norm); per layer the batched LUT6 SwiGLU FFN (RMSNorm
    rows, stacked gate/up projection, silu(g) * u, down projection into the
    residual); then the top-32 of the 262144-row LUT6 LM head for the 32
    hidden states.  Every layer has its own weights, caches and states
    (nothing is re-read from a cache by construction).  The step is timed
    without advancing the lengths, so every repetition does the same work."""
    import numpy as np
    c = CFG
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    H, I, D = c["hidden"], c["inter"], c["head_dim"]
    Hq, Hkv, Hk, Hv, dl = c["n_heads"], c["n_kv_heads"], c["lin_k_heads"], c["lin_v_heads"], c["lin_dim"]
    B, P, V = 32, 16, 262144

    def randn(*shape, std=1.0, dtype=torch.float32):
        return (torch.randn(*shape, generator=g, device=dev) * std).to(dtype)

    def randbytes(*shape):
        return torch.randint(0, 256, shape, generator=g, device=dev, dtype=torch.uint8)

    rng = np.random.default_rng(seed)
    lens = rng.integers(256, 16385, B).astype(np.int32)
    npg = (lens + 1 + P - 1) // P          # pages for the cached keys and the new one
    n_pages = int(npg.sum())
    max_pages = int(npg.max())
    layers = (anelm.BatchLayer * c["layers"])()
    keep, kv_bytes, dn_bytes = [], 0, 0
    for i in range(c["layers"]):
        L = layers[i]
        t = {"ffn_norm_w": 1 + randn(H, std=0.02),
             "gate_up_w": randbytes(2 * I, H * 3 // 4),
             "gate_up_lut": randn(2 * I // 32, 64, std=0.02, dtype=torch.float16),
             "down_w": randbytes(H, I * 3 // 4),
             "down_lut": randn(H // 32, 64, std=0.02, dtype=torch.float16)}
        if (i + 1) % 4 == 0:
            L.kind = anelm.LAYER_ATTENTION
            perm = rng.permutation(n_pages).astype(np.int32)
            table = np.zeros((B, max_pages), np.int32)
            off = 0
            for sq in range(B):
                table[sq, :npg[sq]] = perm[off:off + npg[sq]]
                off += npg[sq]
            t["k_pages"] = randn(n_pages, Hkv, P, D, dtype=torch.float16)
            t["v_pages"] = randn(n_pages, Hkv, P, D, dtype=torch.float16)
            t["page_table"] = torch.from_numpy(table).to(dev)
            t["q_gate"] = randn(B, Hq, 2 * D)
            t["k"] = randn(B, Hkv, D)
            t["v"] = randn(B, Hkv, D)
            t["q_norm_w"] = 1 + randn(D, std=0.02)
            t["k_norm_w"] = 1 + randn(D, std=0.02)
            t["core_out"] = torch.empty(B, Hq * D, device=dev)
            kv_bytes += int(lens.sum() + B) * Hkv * D * 2 * 2
        else:
            L.kind = anelm.LAYER_DELTANET
            L.dn_flags = 1 | 4
            t["state"] = randn(B, Hv, dl, dl, std=0.1)
            t["dn_q"] = randn(B, Hk, dl)
            t["dn_k"] = randn(B, Hk, dl)
            t["dn_v"] = randn(B, Hv, dl)
            t["dn_a"], t["dn_b"] = randn(B, Hv), randn(B, Hv)
            t["dn_A"] = torch.exp(torch.rand(Hv, generator=g, device=dev) * math.log(16.0))
            t["dn_dt_bias"] = randn(Hv)
            t["dn_z"] = randn(B, Hv, dl)
            t["dn_norm_w"] = 1 + randn(dl, std=0.02)
            t["core_out"] = torch.empty(B, Hv * dl, device=dev)
            dn_bytes += B * Hv * dl * dl * 4 * 2
        for name, ten in t.items():
            setattr(L, name, ten.data_ptr())
        keep.append(t)
    lm = (randbytes(V, H * 3 // 4), randn(V // 32, 64, std=0.02, dtype=torch.float16))
    fnorm = 1 + randn(H, std=0.02)
    lens_d = torch.from_numpy(lens).to(dev)
    rope = anelm.ops.rope_table(c["rot_dim"], 16385, c["theta"], dev)
    x = randn(B, H)
    top_idx = torch.empty(B, 32, dtype=torch.int32, device=dev)
    top_val = torch.empty(B, 32, device=dev)
    seqs = anelm.BatchSeqs()
    seqs.n_seqs, seqs.seq_lens, seqs.positions = B, lens_d.data_ptr(), None
    seqs.page_size, seqs.n_pages, seqs.max_pages, seqs.max_seq_len = P, n_pages, max_pages, max_pages * P
    seqs.rope_table, seqs.rope_rows = rope.data_ptr(), 16385
    seqs.final_norm_w, seqs.lm_w, seqs.lm_lut = fnorm.data_ptr(), lm[0].data_ptr(), lm[1].data_ptr()
    seqs.vocab, seqs.top_k, seqs.top_idx, seqs.top_val = V, 32, top_idx.data_ptr(), top_val.data_ptr()
    dims = anelm.HybridDims(H, I, Hq, Hkv, D, c["rot_dim"], 0, c["theta"], c["eps"], Hk, Hv, dl)
    handle = ctypes.c_void_p()
    anelm.call("anelm_batch_step_create", ctypes.byref(handle), ctypes.byref(dims), layers, c["layers"],
               ctypes.byref(seqs), ctypes.c_void_p(x.data_ptr()))
    try:
        us = _gpu_us(torch, lambda: anelm.call("anelm_batch_step_run", handle, 0,
                                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                     reps, warm=1)
    finally:
        anelm.call("anelm_batch_step_destroy", handle)
    w_bytes = c["layers"] * (3 * H * I * 3 // 4 + (2 * I // 32 + H // 32) * 128)
    lm_bytes = V * H * 3 // 4 + (V // 32) * 128
    total = kv_bytes + dn_bytes + w_bytes + lm_bytes
    r = _hbm(us, total)
    r.update({"sequences": B, "sum_len": int(lens.sum()), "kv_bytes": kv_bytes, "deltanet_state_bytes": dn_bytes,
              "lut6_ffn_bytes": w_bytes, "lm_head_bytes": lm_bytes,
              "composition": "fused paged attention step (norms, RoPE, page append, attention, gate), "
                             "batched DeltaNet, batched LUT6 FFN, final norm + LM-head top-32"})
    return r


def measure_step_08b(anelm, torch, dev, reps=50):
    """The same decode step at the reference's default 0.8B shape (24 layers,
    ctx 8192) as one persistent launch; on the 256-CU grid its 2 kv heads and
    16 value heads occupy 128 workgroups in the cores."""
    handle, keep, x, mode = build_step(anelm, torch, dev, seed=5, mode=anelm.STEP_PERSISTENT | anelm.STEP_STATIC,
                                       c=CFG_08B)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for _ in range(5):
        anelm.call("anelm_hybrid_step_run", handle, s)
    us = _gpu_us(torch, lambda: anelm.call("anelm_hybrid_step_run", handle, s), reps, warm=0)
    st = ctypes.c_int(0)
    anelm.call("anelm_hybrid_step_status", handle, ctypes.byref(st))
    assert st.value == 0 and torch.isfinite(x).all(), "0.8B step failed"
    anelm.call("anelm_hybrid_step_destroy", handle)
    del keep
    r = _hbm(us, step_bytes(CFG_08B)["total"])
    r["execution"] = "persistent kernel, one launch per step"
    r["composition"] = ("24 layers: 6 full-attention cores (8q/2kv, ctx 8192), 18 Gated-DeltaNet cores "
                        "(16k/16v heads), 24 LUT6 SwiGLU FFN 1024->3584->1024")
    return r


def measure_complete_step(anelm, torch, dev, reps=20):
    """The same 32-layer step with the projections around the cores inside
    (qwen3_5.cpp:1287-1354 per layer: input norm + LUT6 first projection, the
    DeltaNet conv ring, the core, o_proj + residual, the FFN), as a HIP-graph
    replay of the per-layer launches."""
    handle, keep, x, mode = build_step(anelm, torch, dev, seed=3, mode=anelm.STEP_GRAPH, proj=True)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for _ in range(3):
        anelm.call("anelm_hybrid_step_run", handle, s)
    us = _gpu_us(torch, lambda: anelm.call("anelm_hybrid_step_run", handle, s), reps, warm=0)
    assert torch.isfinite(x).all(), "non-finite hidden state (complete step)"
    anelm.call("anelm_hybrid_step_destroy", handle)
    del keep
    nbytes = step_bytes()["total"] + proj_bytes()
    r = _hbm(us, nbytes)
    r["execution"] = "hip graph replay of the per-layer launches"
    r["composition"] = ("per layer: input norm + LUT6 first projection (2560->12352 DeltaNet, 2560->10240 "
                        "attention), conv ring + DeltaNet core or attention core, LUT6 o_proj 4096->2560 + "
                        "residual, LUT6 SwiGLU FFN")
    return r


def cpu_baselines_per_config(seconds=1.0):
    """The oracle (single-threaded C restatement of cpu_ops) on each other
    workload, each on a bounded sample of about `seconds`:
    C1 one 0.8B-shaped attention decode over 513 keys; C2 one 16-head DeltaNet
    step; C3a causal prefill at 4096 tokens from the last 16 rows (cost per
    (row, key) pair x S(S+1)/2); C3b chunked-DeltaNet prefill from a 128-token
    prefix (x 32: the recurrence is sequential per token); C5 the 32-sequence
    step composed from timed units (attention per cached key, one 32-head
    DeltaNet step, one FFN block, one 8192-row LM-head slice) over the drawn
    lengths."""
    import numpy as np
    from workloads import attn_decode_case, deltanet_case, load_oracle, lut6_matrix, prefill_inputs
    orc = load_oracle()
    orc.use_timing_build()

    def med(fn):
        fn()
        ts = []
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end or len(ts) < 3:
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts) * 1e6, len(ts)

    res = {}
    c = attn_decode_case(11)
    kc32 = np.ascontiguousarray(c.k_cache[:c.length + 1].astype(np.float32))   # the reference's fp32 ring
    vc32 = np.ascontiguousarray(c.v_cache[:c.length + 1].astype(np.float32))
    qg = c.q_gate.reshape(8, 2, 256)

    def c1():   # qwen3_5.cpp:944-1002 on an fp32 ring of 513 keys
        qn = orc.rmsnorm(qg[:, 0], c.q_norm_w)
        kn = orc.rmsnorm(c.k, c.k_norm_w)
        qn, kn = orc.apply_rope(qn, kn, 8, 2, 256, 256, 256, 64, c.pos, c.theta)
        kc32[c.length] = kn
        o = orc.gqa_attention(qn, kc32, vc32, 8, 2, 256, 256, 0, c.length + 1, c.length + 1)
        return orc.mul_sigmoid(o, qg[:, 1])
    us, n = med(c1)
    res["decode_attention_0.8b"] = {"us": round(us, 1), "sample": f"median of {n} calls (fp32 ring, 513 keys)"}
    d = deltanet_case(12, Hk=16, Hv=16)
    us, n = med(lambda: orc.deltanet_decode(d.state, d.q, d.k, d.v, d.a, d.b, d.A, d.dt_bias, 0))
    res["deltanet_decode"] = {"us": round(us, 1), "sample": f"median of {n} calls"}
    S = 4096
    q, k, v = prefill_inputs(13, S, 16, 4, 256)
    us, n = med(lambda: orc.prefill_attention(q, k, v, S - 16, S))
    pairs = sum(t + 1 for t in range(S - 16, S))
    res["prefill_attention_4096"] = {"us": round(us / pairs * S * (S + 1) / 2, 1),
                                     "sample": f"rows {S - 16}..{S - 1} (median of {n}), x S(S+1)/2 pairs"}
    d = deltanet_case(14, Hk=16, Hv=32, S=128)
    us, n = med(lambda: orc.deltanet_prefill(d.state, d.q, d.k, d.v, d.a, d.b, d.A, d.dt_bias, 1))
    res["deltanet_prefill_4096"] = {"us": round(us * S / 128, 1), "sample": f"128 tokens (median of {n}) x 32"}
    # C5 units
    L0 = 4096
    kc = np.random.default_rng(15).standard_normal((L0, 4, 256)).astype(np.float32)
    qq = np.random.default_rng(16).standard_normal((16, 512)).astype(np.float32)
    u_key, _ = med(lambda: orc.gqa_attention(qq, kc, kc, 16, 4, 256, 512, 0, L0, L0))
    d = deltanet_case(17, Hk=16, Hv=32)
    u_dn, _ = med(lambda: orc.deltanet_decode(d.state, d.q, d.k, d.v, d.a, d.b, d.A, d.dt_bias, 5, d.z, d.norm_w))
    g, u, dn = lut6_matrix(18, 9216, 2560), lut6_matrix(19, 9216, 2560), lut6_matrix(20, 2560, 9216)
    xx = np.random.default_rng(21).standard_normal(2560).astype(np.float32)
    u_ffn, _ = med(lambda: orc.lut6_ffn(xx, g[:2], u[:2], dn[:2], 2560, 9216))
    lm = lut6_matrix(22, 8192, 2560)
    u_lm, _ = med(lambda: orc.lut6_matvec(lm[0], lm[1], xx, 8192, 2560))
    lens = np.random.default_rng(12).integers(256, 16385, 32)   # the GPU step's draw
    step = (8 * u_key / L0 * float(lens.sum()) + 24 * 32 * u_dn + 32 * 32 * u_ffn + 32 * (262144 / 8192) * u_lm)
    res["batch32_decode_step"] = {"us": round(step, 1),
                                  "sample": "units timed (attention over 4096 fp32 keys, 32-head DeltaNet step, "
                                            "one FFN block, 8192-row LM-head slice), composed over the drawn "
                                            "lengths x 32 sequences x 32 layers"}
    return res


def cpu_baseline(seconds=12.0):
    """The oracle (a single-threaded C restatement of the reference cpu_ops
    path) on a bounded sample of the same step: one block of four layers
    (1 attention over an fp32 8192-key cache as the reference stores it,
    3 DeltaNet, 4 LUT6 FFN blocks evaluated as dequantise + fp32 matvec),
    repeated for about `seconds`, scaled x8 to the 32-layer step."""
    import numpy as np
    from workloads import load_oracle
    orc = load_oracle()
    orc.use_timing_build()
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
                      f"oracle/anelm_oracle.c built -O3 -march=x86-64-v3 with vectorised reductions "
                      f"(liboracle_timing.so), 1 thread, {cpu_model}, nproc {os.cpu_count()}"}


def trace_step(runs=3, save=None):
    """Phase timeline of the persistent step from libanelm_trace.so (the same
    library built with the step's clock stamps compiled in): per phase kind
    (DeltaNet core, attention core, gate/up, down) the median over layers of
    the workgroup-median compute time, the spread of barrier arrivals, and the
    time from the last arrival to the median workgroup seeing the release
    (plus the gap from release to the next phase's compute start)."""
    import numpy as np
    import torch
    from workloads import load_package
    pkg_dir = os.path.join(ROOT, "ane-lm_amd")
    trace_lib = os.path.join(pkg_dir, "libanelm_trace.so")
    if not os.path.exists(trace_lib):
        raise SystemExit(f"{trace_lib} not built (make -C ane-lm_amd/csrc)")
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "ane_lm_amd", os.path.join(pkg_dir, "__init__.py"), submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ane_lm_amd"] = mod
    spec.loader.exec_module(mod)
    mod.LIB_PATH = trace_lib
    anelm = load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream()
    out = []
    with torch.cuda.stream(stream):
        handle, keep, x, mode = build_step(anelm, torch, dev, mode=anelm.STEP_PERSISTENT | anelm.STEP_STATIC)
        s = ctypes.c_void_p(stream.cuda_stream)
        for _ in range(5):
            anelm.call("anelm_hybrid_step_run", handle, s)
        grid, rows = 256, 193
        for r in range(runs):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            anelm.call("anelm_hybrid_step_run", handle, s)
            e1.record(stream)
            torch.cuda.synchronize()
            buf = np.zeros(1024 * 193 * 8, dtype=np.uint64)
            g, ph = ctypes.c_int(0), ctypes.c_int(0)
            anelm.call("anelm_hybrid_step_trace", handle, ctypes.c_void_p(buf.ctypes.data), buf.size,
                       ctypes.byref(g), ctypes.byref(ph))
            grid, rows = g.value, ph.value
            out.append((e0.elapsed_time(e1) * 1e3, buf[: grid * rows * 8].reshape(grid, rows, 8).astype(np.int64)))
        st = ctypes.c_int(0)
        anelm.call("anelm_hybrid_step_status", handle, ctypes.byref(st))
        assert st.value == 0, "a grid barrier of the persistent step timed out"
        anelm.call("anelm_hybrid_step_destroy", handle)
    n_layers = CFG["layers"]
    tick_us = 0.01   # 100 MHz real-time clock
    kinds = {"deltanet_core": [], "attention_split": [], "attention_merge": [], "gate_up": [], "down": []}
    # phases in execution order: core, (attention: merge), gate/up, down
    seq = []
    for layer in range(n_layers):
        att = (layer + 1) % 4 == 0
        seq.append((3 * layer, "attention_split" if att else "deltanet_core"))
        if att:
            seq.append((3 * n_layers + layer // 4, "attention_merge"))
        seq.append((3 * layer + 1, "gate_up"))
        seq.append((3 * layer + 2, "down"))
    runs_out = []
    for us, tr in out:
        t0 = tr[:, rows - 1, 0].min()
        t_end = tr[:, rows - 1, 1].max()
        S, E, A, R = (tr[:, :rows - 1, k] - t0 for k in range(4))
        for q, (p, kind) in enumerate(seq):
            comp = np.median(E[:, p] - S[:, p]) * tick_us
            arr_spread = (A[:, p].max() - np.median(A[:, p])) * tick_us
            last_arr = A[:, p].max()
            if q + 1 < len(seq):
                pn = seq[q + 1][0]
                rel = (np.median(R[:, p]) - last_arr) * tick_us
                nxt = (np.median(S[:, pn]) - np.median(R[:, p])) * tick_us
                period = (np.median(S[:, pn]) - np.median(S[:, p])) * tick_us
            else:
                rel, nxt = 0.0, 0.0
                period = (t_end - t0 - np.median(S[:, p])) * tick_us
            kinds[kind].append((comp, arr_spread, rel, nxt, period))
        runs_out.append({"event_us": round(us, 2), "clock_us": round((t_end - t0) * tick_us, 2)})
    summary = {}
    for kind, v in kinds.items():
        a = np.array(v)
        summary[kind] = {"phases": int(len(a) // runs),
                         "compute_us": round(float(np.median(a[:, 0])), 2),
                         "arrival_spread_us": round(float(np.median(a[:, 1])), 2),
                         "last_arrival_to_release_us": round(float(np.median(a[:, 2])), 2),
                         "release_to_next_start_us": round(float(np.median(a[:, 3])), 2),
                         "phase_period_us": round(float(np.median(a[:, 4])), 2)}
    per_layer = {k: round(summary[k]["phase_period_us"], 2) for k in summary}
    if save:
        import numpy as np
        np.savez_compressed(save, *[tr for _, tr in out])
    print(json.dumps({"trace": "persistent step phase timeline (median over layers of each phase kind)",
                      "runs": runs_out, "phases": summary, "period_us": per_layer}, indent=1))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--mode", choices=["persistent", "graph", "eager"], default=None,
                    help="decode-step execution (default: persistent, else graph)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-cores", action="store_true",
                    help="do not time the other workloads (decode/prefill attention, DeltaNet, batched decode)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                    help="after the timed steps, copy MB MiB device-to-device once (a kernel of known "
                         "traffic that scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--trace-step", action="store_true",
                    help="print the persistent step's phase timeline from libanelm_trace.so instead")
    ap.add_argument("--trace-save", default=None, metavar="NPZ",
                    help="with --trace-step: also save the raw stamps [grid][phases+1][4] per run")
    args = ap.parse_args()
    if args.trace_step:
        trace_step(save=args.trace_save)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this benchmark measures one GPU; the decode step does not "
                                   "shard across GPUs here (run with --gpus 1)"}))
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
        del keep
        torch.cuda.empty_cache()
        cores = None if args.skip_cores else measure_cores(anelm, torch, dev)
        if cores is not None:
            torch.cuda.empty_cache()
            cores["batch32_decode_step"] = measure_batch32_step(anelm, torch, dev)
            torch.cuda.empty_cache()
            cores["complete_step_graph"] = measure_complete_step(anelm, torch, dev)
            cores["decode_step_0.8b"] = measure_step_08b(anelm, torch, dev)

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
    if cores is not None:
        result["cores"] = cores
    if not args.skip_cpu:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        if cores is not None:
            # the same oracle, one thread, beside each other workload's GPU time
            per = cpu_baselines_per_config()
            for name, v in per.items():
                if name in cores:
                    cores[name]["cpu_us"] = v["us"]
                    cores[name]["cpu_sample"] = v["sample"]
    print(json.dumps(result))


if __name__ == "__main__":
    main()
