"""Seeded synthetic inputs for the benchmark configurations, plus loaders for
the product package and the oracle.

Used by tests/, bench.py and __graft_entry__.smoke().  Values that the
kernels consume as fp16 are drawn in fp32, rounded to fp16 first, and the
oracle receives their exact fp32 widening.
"""
from __future__ import annotations

import importlib.util
import math
import os
import sys
from dataclasses import dataclass

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_package():
    """Imports ane-lm_amd/ as module `ane_lm_amd` (raises if libanelm.so is absent)."""
    if "ane_lm_amd" in sys.modules:
        return sys.modules["ane_lm_amd"]
    pkg_dir = os.path.join(ROOT, "ane-lm_amd")
    spec = importlib.util.spec_from_file_location(
        "ane_lm_amd", os.path.join(pkg_dir, "__init__.py"), submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ane_lm_amd"] = mod
    spec.loader.exec_module(mod)
    mod.lib()
    return mod


def load_oracle():
    """Imports oracle/oracle.py as module `anelm_oracle` (the checker)."""
    if "anelm_oracle" in sys.modules:
        return sys.modules["anelm_oracle"]
    path = os.path.join(ROOT, "oracle", "oracle.py")
    spec = importlib.util.spec_from_file_location("anelm_oracle", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules["anelm_oracle"] = mod
    spec.loader.exec_module(mod)
    mod.lib()
    return mod


def f16(x):
    """Rounds to fp16 (numpy RNE) and returns the uint16 bit patterns."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def widen(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


# ------------------------------------------------------------- attention
@dataclass
class AttnDecodeCase:
    n_heads: int
    n_kv_heads: int
    head_dim: int
    rot_dim: int
    pos: int
    theta: float
    eps: float
    capacity: int
    start: int
    length: int
    q_gate: np.ndarray   # [Hq][2D] fp32
    k: np.ndarray        # [Hkv][D]
    v: np.ndarray
    k_cache: np.ndarray  # [cap][Hkv][D] uint16 (fp16 bits)
    v_cache: np.ndarray
    q_norm_w: np.ndarray
    k_norm_w: np.ndarray


def attn_decode_case(seed, n_heads=8, n_kv_heads=2, head_dim=256, cached=512, capacity=None,
                     start=0, rot_dim=None, theta=1e7, eps=1e-6, pos=None):
    """Full-attention decode step inputs (the 0.8B-shaped step by default:
    8 q / 2 kv heads, D 256, 512 cached fp16 keys, position 512)."""
    rng = np.random.default_rng(seed)
    D = head_dim
    capacity = max(cached + 1, 2048) if capacity is None else capacity
    rot_dim = D // 4 if rot_dim is None else rot_dim
    pos = cached if pos is None else pos
    kc = np.zeros((capacity, n_kv_heads, D), np.uint16)
    vc = np.zeros((capacity, n_kv_heads, D), np.uint16)
    slots = (start + np.arange(cached)) % capacity
    kc[slots] = f16(rng.standard_normal((cached, n_kv_heads, D)))
    vc[slots] = f16(rng.standard_normal((cached, n_kv_heads, D)))
    return AttnDecodeCase(
        n_heads, n_kv_heads, D, rot_dim, pos, theta, eps, capacity, start, cached,
        rng.standard_normal((n_heads, 2 * D)).astype(np.float32),
        rng.standard_normal((n_kv_heads, D)).astype(np.float32),
        rng.standard_normal((n_kv_heads, D)).astype(np.float32),
        kc, vc,
        (1.0 + 0.02 * rng.standard_normal(D)).astype(np.float32),
        (1.0 + 0.02 * rng.standard_normal(D)).astype(np.float32))


def prefill_inputs(seed, S, Hq, Hkv, D):
    """Causal prefill inputs: fp16 q [S][Hq][D], k/v [S][Hkv][D] ~ N(0,1)."""
    rng = np.random.default_rng(seed)
    return (f16(rng.standard_normal((S, Hq, D))), f16(rng.standard_normal((S, Hkv, D))),
            f16(rng.standard_normal((S, Hkv, D))))


# -------------------------------------------------------------- DeltaNet
@dataclass
class DeltaNetCase:
    state: np.ndarray   # [Hv][dk][dv]
    q: np.ndarray       # [..., Hk, dk]
    k: np.ndarray
    v: np.ndarray       # [..., Hv, dv]
    a: np.ndarray       # [..., Hv]
    b: np.ndarray
    A: np.ndarray       # [Hv] = exp(A_log)
    dt_bias: np.ndarray
    z: np.ndarray       # [Hv, dv] (gated-norm epilogue input)
    norm_w: np.ndarray  # [dv]


def deltanet_case(seed, Hk=16, Hv=16, dk=128, dv=128, S=None):
    """DeltaNet inputs: state ~ N(0, 0.1); q, k ~ N(0,1) then l2-normalised;
    v ~ N(0,1); beta = sigmoid(N(0,1)); a ~ N(0,1); A_log ~ U(0, ln 16);
    dt_bias ~ N(0,1) (the workload leaves dt_bias open; N(0,1) is this choice).
    S=None gives one decode step, else S tokens."""
    rng = np.random.default_rng(seed)
    lead = () if S is None else (S,)

    def l2n(x):
        return (x / np.sqrt((x.astype(np.float64) ** 2).sum(-1, keepdims=True))).astype(np.float32)

    return DeltaNetCase(
        (0.1 * rng.standard_normal((Hv, dk, dv))).astype(np.float32),
        l2n(rng.standard_normal(lead + (Hk, dk))),
        l2n(rng.standard_normal(lead + (Hk, dk))),
        rng.standard_normal(lead + (Hv, dv)).astype(np.float32),
        rng.standard_normal(lead + (Hv,)).astype(np.float32),
        rng.standard_normal(lead + (Hv,)).astype(np.float32),
        np.exp(rng.uniform(0.0, math.log(16.0), Hv)).astype(np.float32),
        rng.standard_normal(Hv).astype(np.float32),
        rng.standard_normal((Hv, dv)).astype(np.float32),
        (1.0 + 0.02 * rng.standard_normal(dv)).astype(np.float32))


# ------------------------------------------------------------------ LUT6
def pack_lut6(idx):
    """Packs 6-bit indices (any shape, last axis % 4 == 0) 4 per 3 bytes, LSB first."""
    idx = np.asarray(idx, np.uint32)
    g = idx.reshape(-1, 4)
    w = g[:, 0] | (g[:, 1] << 6) | (g[:, 2] << 12) | (g[:, 3] << 18)
    out = np.stack([w & 0xff, (w >> 8) & 0xff, (w >> 16) & 0xff], axis=1).astype(np.uint8)
    return out.reshape(idx.shape[:-1] + (idx.shape[-1] * 3 // 4,))


def lut6_matrix(seed, out_dim, in_dim, lut_std=0.02):
    """Random LUT6 matrix: indices U[0,64), one fp16 LUT ~ N(0, lut_std) per 32 rows.
    Returns (packed [out][in*3/4] uint8, lut [out/32][64] uint16, idx)."""
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, 64, (out_dim, in_dim), dtype=np.uint8)
    lut = f16(lut_std * rng.standard_normal((out_dim // 32, 64)))
    return pack_lut6(idx), lut, idx


def lut6_dense(idx, lut):
    """Dequantised fp32 weights (exact: fp16 LUT values widen exactly)."""
    out_dim = idx.shape[0]
    lutf = widen(lut)
    return lutf[np.arange(out_dim)[:, None] // 32, idx]


# -------------------------------------------------------------- the 4B step
QWEN35_4B = dict(hidden=2560, inter=9216, layers=32, n_heads=16, n_kv_heads=4, head_dim=256,
                 rot_dim=64, theta=1e7, eps=1e-6, lin_k_heads=16, lin_v_heads=32, lin_dim=128,
                 full_attention_interval=4)
QWEN35_08B = dict(hidden=1024, inter=3584, layers=24, n_heads=8, n_kv_heads=2, head_dim=256,
                  rot_dim=64, theta=1e7, eps=1e-6, lin_k_heads=16, lin_v_heads=16, lin_dim=128,
                  full_attention_interval=4)


def layer_is_attention(i, interval=4):
    """models/llm/qwen3_5.cpp:64-71: layer i is full attention when (i+1) % interval == 0."""
    return (i + 1) % interval == 0


# ------------------------------------------------- hybrid decode step model
@dataclass
class HybridModel:
    """Seeded random-init weights and state of a Qwen3.5-shaped hybrid stack
    (layer i is full attention iff (i+1) % 4 == 0), host copies in numpy."""
    dims: dict
    layers: list          # per layer dict of numpy arrays / ints
    x: np.ndarray         # [hidden] fp32


def hybrid_model(seed, n_layers, dims=QWEN35_4B, rings=None, cap=8192, lut_std=0.02):
    """rings: per attention layer (start, len); default (0, 700).  Cached keys
    and values are fp16 ~ N(0,1); weights as the benchmark describes."""
    rng = np.random.default_rng(seed)
    d = dims
    H, I, D = d["hidden"], d["inter"], d["head_dim"]
    Hq, Hkv, Hk, Hv, dl = d["n_heads"], d["n_kv_heads"], d["lin_k_heads"], d["lin_v_heads"], d["lin_dim"]
    layers = []
    n_attn = 0

    def lut(rows):
        return f16(lut_std * rng.standard_normal((rows // 32, 64)))

    def lw(rows, cols):
        return rng.integers(0, 256, (rows, cols * 3 // 4), dtype=np.uint8)

    for i in range(n_layers):
        L = {}
        if layer_is_attention(i):
            start, length = (rings[n_attn] if rings else (0, 700))
            n_attn += 1
            L["kind"] = 1
            L["q_gate"] = rng.standard_normal((Hq, 2 * D)).astype(np.float32)
            L["k"] = rng.standard_normal((Hkv, D)).astype(np.float32)
            L["v"] = rng.standard_normal((Hkv, D)).astype(np.float32)
            L["k_cache"] = f16(rng.standard_normal((cap, Hkv, D)))
            L["v_cache"] = f16(rng.standard_normal((cap, Hkv, D)))
            L["q_norm_w"] = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
            L["k_norm_w"] = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
            L["start"], L["len"], L["cap"], L["pos"] = start, length, cap, length
        else:
            dn = deltanet_case(int(rng.integers(1 << 30)), Hk=Hk, Hv=Hv, dk=dl, dv=dl)
            L["kind"] = 0
            L.update(state=dn.state, dn_q=dn.q, dn_k=dn.k, dn_v=dn.v, dn_a=dn.a, dn_b=dn.b,
                     dn_A=dn.A, dn_dt_bias=dn.dt_bias, dn_z=dn.z, dn_norm_w=dn.norm_w)
            L["dn_flags"] = 1 | 4
        L["ffn_norm_w"] = (1 + 0.02 * rng.standard_normal(H)).astype(np.float32)
        L["gate_w"], L["gate_lut"] = lw(I, H), lut(I)
        L["up_w"], L["up_lut"] = lw(I, H), lut(I)
        L["down_w"], L["down_lut"] = lw(H, I), lut(H)
        layers.append(L)
    return HybridModel(dict(d), layers, rng.standard_normal(H).astype(np.float32))


def oracle_hybrid_step(orc, m: HybridModel):
    """One decode step through the oracle (models/llm/qwen3_5.cpp:1278-1356 over
    the cores): per layer the attention or DeltaNet core, then
    x += lut6_ffn(rmsnorm(x)).  Updates m in place (x, states, caches, rings)
    and returns the per-layer core outputs."""
    d = m.dims
    H, I, D = d["hidden"], d["inter"], d["head_dim"]
    outs = []
    for L in m.layers:
        if L["kind"] == 1:
            out, kc, vc, st, ln = orc.full_attn_decode(
                L["q_gate"], L["k"], L["v"], L["k_cache"], L["v_cache"], L["q_norm_w"], L["k_norm_w"],
                d["n_heads"], d["n_kv_heads"], D, d["rot_dim"], L["pos"], d["theta"], d["eps"], 0, True,
                L["start"], L["len"], L["cap"])
            L["k_cache"], L["v_cache"], L["start"], L["len"] = kc, vc, st, ln
            L["pos"] += 1
            outs.append(out.reshape(-1))
        else:
            y, S = orc.deltanet_decode(L["state"], L["dn_q"], L["dn_k"], L["dn_v"], L["dn_a"], L["dn_b"],
                                       L["dn_A"], L["dn_dt_bias"], L["dn_flags"], L["dn_z"], L["dn_norm_w"])
            L["state"] = S
            outs.append(y.reshape(-1))
        n = orc.rmsnorm(m.x, L["ffn_norm_w"], d["eps"])
        m.x = (m.x + orc.lut6_ffn(n, (L["gate_w"], L["gate_lut"]), (L["up_w"], L["up_lut"]),
                                  (L["down_w"], L["down_lut"]), H, I)).astype(np.float32)
    return outs
