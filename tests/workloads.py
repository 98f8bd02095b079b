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
    """Imports oracle/oracle.py as module `anelm_oracle` (the oracle)."""
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


def hybrid_model(seed, n_layers, dims=QWEN35_4B, rings=None, cap=8192, lut_std=0.02, dn_flags=1 | 4):
    """rings: per attention layer (start, len); default (0, 700).  Cached keys
    and values are fp16 ~ N(0,1); weights as the benchmark describes;
    dn_flags for every DeltaNet layer (ANELM_DN_* bits)."""
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
            L["dn_flags"] = dn_flags
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


# ------------------------------------------------ greedy decode of a tiny LM
TINY_LM = dict(hidden=1024, inter=2048, layers=4, n_heads=8, n_kv_heads=2, head_dim=256, rot_dim=64,
               theta=1e7, eps=1e-6, lin_k_heads=16, lin_v_heads=16, lin_dim=128, conv_kernel=4,
               vocab=4096, cap=128)


def tiny_lm(seed, dims=TINY_LM, lut_std=0.02):
    """Seeded random-init Qwen3.5-shaped hybrid LM (layer i is full attention
    iff (i+1) % 4 == 0) with every projection LUT6-palettised, as the
    reference's CoreML path stores them (scripts/export_hybrid_chunks.py:42):
    per layer input/post norms, the first projection (DeltaNet: qkv | z | a | b,
    attention: q_gate | k | v; models/llm/qwen3_5.cpp:849-910, 944-1002), the
    DeltaNet conv1d weights, A = exp(A_log) and dt_bias, o_proj and the SwiGLU
    FFN; an fp32 embedding table, a final norm and a LUT6 LM head."""
    rng = np.random.default_rng(seed)
    d = dims
    H, I, V = d["hidden"], d["inter"], d["vocab"]
    Hq, Hkv, D = d["n_heads"], d["n_kv_heads"], d["head_dim"]
    Hk, Hv, dl = d["lin_k_heads"], d["lin_v_heads"], d["lin_dim"]
    qkv = 2 * Hk * dl + Hv * dl

    def norm_w(n):
        return (1.0 + 0.02 * rng.standard_normal(n)).astype(np.float32)

    def lut6(out_dim, in_dim):
        idx = rng.integers(0, 64, (out_dim, in_dim), dtype=np.uint8)
        lut = f16(lut_std * rng.standard_normal((out_dim // 32, 64)))
        return pack_lut6(idx), lut

    layers = []
    for i in range(d["layers"]):
        L = dict(attn=layer_is_attention(i), in_norm=norm_w(H), post_norm=norm_w(H))
        if L["attn"]:
            L["first"] = lut6(Hq * 2 * D + 2 * Hkv * D, H)
            L["q_norm"], L["k_norm"] = norm_w(D), norm_w(D)
            L["o"] = lut6(H, Hq * D)
        else:
            L["first"] = lut6(qkv + Hv * dl + 2 * Hv, H)
            L["conv_w"] = (0.5 * rng.standard_normal((qkv, d["conv_kernel"]))).astype(np.float32)
            L["A"] = np.exp(rng.uniform(0.0, math.log(16.0), Hv)).astype(np.float32)
            L["dt_bias"] = rng.standard_normal(Hv).astype(np.float32)
            L["norm_w"] = norm_w(dl)
            L["o"] = lut6(H, Hv * dl)
        L["gate"], L["up"], L["down"] = lut6(I, H), lut6(I, H), lut6(H, I)
        layers.append(L)
    return dict(dims=d, layers=layers, embed=rng.standard_normal((V, H)).astype(np.float32),
                final_norm=norm_w(H), lm_head=lut6(V, H))


class OracleLM:
    """Decode loop of the tiny LM on the oracle: Qwen35Model::forward
    (models/llm/qwen3_5.cpp:1278-1417) -- embedding, per layer RMSNorm, first
    projection, DeltaNet core (conv1d + SiLU, :867-875, then :879-908) or
    attention core (:944-1002), o_proj and residual, RMSNorm + SwiGLU FFN and
    residual; final norm, LM head, and the greedy rule of core/sampling.cpp:47-53
    (first maximum)."""

    def __init__(self, orc, m):
        self.orc, self.m = orc, m
        d = m["dims"]
        self.st = []
        for L in m["layers"]:
            if L["attn"]:
                shape = (d["cap"], d["n_kv_heads"], d["head_dim"])
                self.st.append(dict(kc=np.zeros(shape, np.uint16), vc=np.zeros(shape, np.uint16), start=0, len=0))
            else:
                qkv = 2 * d["lin_k_heads"] * d["lin_dim"] + d["lin_v_heads"] * d["lin_dim"]
                self.st.append(dict(conv=np.zeros((qkv, d["conv_kernel"] - 1), np.float32), cpos=0,
                                    S=np.zeros((d["lin_v_heads"], d["lin_dim"], d["lin_dim"]), np.float32)))

    def step(self, token, pos):
        orc, m, d = self.orc, self.m, self.m["dims"]
        H, I = d["hidden"], d["inter"]
        Hk, Hv, dl = d["lin_k_heads"], d["lin_v_heads"], d["lin_dim"]
        x = m["embed"][token].copy()
        for L, s in zip(m["layers"], self.st):
            xn = orc.rmsnorm(x, L["in_norm"], d["eps"])
            fw, fl = L["first"]
            proj = orc.lut6_matvec(fw, fl, xn, fl.shape[0] * 32, H)
            if L["attn"]:
                Hq, Hkv, D = d["n_heads"], d["n_kv_heads"], d["head_dim"]
                qg = proj[:Hq * 2 * D].reshape(Hq, 2 * D)
                k = proj[Hq * 2 * D:Hq * 2 * D + Hkv * D].reshape(Hkv, D)
                v = proj[Hq * 2 * D + Hkv * D:].reshape(Hkv, D)
                pre, s["kc"], s["vc"], s["start"], s["len"] = orc.full_attn_decode(
                    qg, k, v, s["kc"], s["vc"], L["q_norm"], L["k_norm"], Hq, Hkv, D, d["rot_dim"], pos,
                    d["theta"], d["eps"], 0, True, s["start"], s["len"], d["cap"])
            else:
                qkv = 2 * Hk * dl + Hv * dl
                co, s["conv"], s["cpos"] = orc.conv1d_update(s["conv"], s["cpos"], proj[:qkv], L["conv_w"],
                                                            d["conv_kernel"])
                co = orc.silu(co)
                q = co[:Hk * dl].reshape(Hk, dl)
                k = co[Hk * dl:2 * Hk * dl].reshape(Hk, dl)
                v = co[2 * Hk * dl:].reshape(Hv, dl)
                z = proj[qkv:qkv + Hv * dl].reshape(Hv, dl)
                a = proj[qkv + Hv * dl:qkv + Hv * dl + Hv]
                b = proj[qkv + Hv * dl + Hv:]
                pre, s["S"] = orc.deltanet_decode(s["S"], q, k, v, a, b, L["A"], L["dt_bias"], 1 | 4, z,
                                                  L["norm_w"])
            ow, ol = L["o"]
            x = x + orc.lut6_matvec(ow, ol, pre.reshape(-1), H, pre.size)
            xn = orc.rmsnorm(x, L["post_norm"], d["eps"])
            x = x + orc.lut6_ffn(xn, L["gate"], L["up"], L["down"], H, I)
        xf = orc.rmsnorm(x, m["final_norm"], d["eps"])
        lw, ll = m["lm_head"]
        logits = orc.lut6_matvec(lw, ll, xf, d["vocab"], H)
        return orc.argmax(logits), logits


# ------------------------------------------- batched decode over paged KV
@dataclass
class PagedCase:
    """Sequences over shuffled fp16 pages [page][Hkv][P][D]: sequence s holds
    lens[s] cached keys (key t in page table[s][t // P], row t % P) and one
    page slot for its next key."""
    lens: np.ndarray      # [n_seqs] int32, cached keys before the step
    table: np.ndarray     # [n_seqs][max_pages] int32
    k_pages: np.ndarray   # uint16 fp16 bits
    v_pages: np.ndarray
    page_size: int

    def gather(self, s, pages, n):
        """First n keys of sequence s from `pages` as a contiguous fp32 [n][Hkv][D] cache."""
        P = self.page_size
        pg = self.table[s, :(n + P - 1) // P]
        Hkv, D = pages.shape[1], pages.shape[3]
        return widen(pages[pg]).transpose(0, 2, 1, 3).reshape(-1, Hkv, D)[:n]


def paged_case(seed, n_seqs=32, lo=256, hi=16384, Hkv=4, D=256, P=16, lens=None, spare=1):
    """Ragged lengths U[lo, hi] (seeded), a page for every key including
    `spare` more (the next steps' keys), pages shuffled over the pool, fp16
    K / V ~ N(0,1)."""
    rng = np.random.default_rng(seed)
    lens = (rng.integers(lo, hi + 1, n_seqs) if lens is None else np.asarray(lens)).astype(np.int32)
    npg = (lens + spare + P - 1) // P
    n_pages = int(npg.sum())
    perm = rng.permutation(n_pages).astype(np.int32)
    table = np.zeros((len(lens), int(npg.max())), np.int32)
    off = 0
    for s in range(len(lens)):
        table[s, :npg[s]] = perm[off:off + npg[s]]
        off += npg[s]
    kp = f16(rng.standard_normal((n_pages, Hkv, P, D), dtype=np.float32))
    vp = f16(rng.standard_normal((n_pages, Hkv, P, D), dtype=np.float32))
    return PagedCase(lens, table, kp, vp, P)


@dataclass
class BatchModel:
    """Seeded random-init hybrid stack for a batch of sequences (layer i is
    full attention iff (i+1) % 4 == 0): per attention layer its own page
    pool (PagedCase, shared lengths) and per-sequence q_gate / k / v; per
    DeltaNet layer per-sequence states and inputs with the layer's A,
    dt_bias and norm weights; per layer the FFN with gate and up stacked as
    one [2*inter][hidden] LUT6 projection; x [B][hidden]."""
    dims: dict
    lens: np.ndarray
    layers: list
    x: np.ndarray


def batch_model(seed, n_layers, n_seqs, lo=256, hi=2048, dims=QWEN35_4B, lut_std=0.02, P=16, spare=2):
    rng = np.random.default_rng(seed)
    d = dims
    H, I, D = d["hidden"], d["inter"], d["head_dim"]
    Hq, Hkv, Hk, Hv, dl = d["n_heads"], d["n_kv_heads"], d["lin_k_heads"], d["lin_v_heads"], d["lin_dim"]
    lens = rng.integers(lo, hi + 1, n_seqs).astype(np.int32)
    layers = []

    def l2n(x):
        return (x / np.sqrt((x.astype(np.float64) ** 2).sum(-1, keepdims=True))).astype(np.float32)

    def normal(*shape, std=1.0):
        return (std * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)

    for i in range(n_layers):
        L = {}
        if layer_is_attention(i):
            L["kind"] = 1
            L["pages"] = paged_case(int(rng.integers(1 << 30)), lens=lens, Hkv=Hkv, D=D, P=P, spare=spare)
            L["q_gate"] = normal(n_seqs, Hq, 2 * D)
            L["k"] = normal(n_seqs, Hkv, D)
            L["v"] = normal(n_seqs, Hkv, D)
            L["q_norm_w"] = 1 + normal(D, std=0.02)
            L["k_norm_w"] = 1 + normal(D, std=0.02)
        else:
            L["kind"] = 0
            L["state"] = normal(n_seqs, Hv, dl, dl, std=0.1)
            L["dn_q"] = l2n(normal(n_seqs, Hk, dl))
            L["dn_k"] = l2n(normal(n_seqs, Hk, dl))
            L["dn_v"] = normal(n_seqs, Hv, dl)
            L["dn_a"] = normal(n_seqs, Hv)
            L["dn_b"] = normal(n_seqs, Hv)
            L["dn_A"] = np.exp(rng.uniform(0.0, math.log(16.0), Hv)).astype(np.float32)
            L["dn_dt_bias"] = normal(Hv)
            L["dn_z"] = normal(n_seqs, Hv, dl)
            L["dn_norm_w"] = 1 + normal(dl, std=0.02)
            L["dn_flags"] = 1 | 4
        L["ffn_norm_w"] = 1 + normal(H, std=0.02)
        L["gate_up_w"] = rng.integers(0, 256, (2 * I, H * 3 // 4), dtype=np.uint8)
        L["gate_up_lut"] = f16(lut_std * rng.standard_normal((2 * I // 32, 64)))
        L["down_w"] = rng.integers(0, 256, (H, I * 3 // 4), dtype=np.uint8)
        L["down_lut"] = f16(lut_std * rng.standard_normal((H // 32, 64)))
        layers.append(L)
    return BatchModel(dict(d), lens, layers, normal(n_seqs, H))


class OracleBatch:
    """The oracle's decode step for every sequence of a BatchModel: per
    sequence its attention ring (the gathered pages, capacity for `steps`
    more keys) or DeltaNet state, then the FFN on all rows."""

    def __init__(self, orc, m: BatchModel, steps):
        self.orc, self.m = orc, m
        self.rings = {}
        for i, L in enumerate(m.layers):
            if L["kind"] == 1:
                c = L["pages"]
                rows = []
                for s, n in enumerate(m.lens):
                    cap = int(n) + steps
                    kc = np.zeros((cap,) + c.k_pages.shape[1:2] + c.k_pages.shape[3:], np.uint16)
                    vc = np.zeros_like(kc)
                    kc[:n], vc[:n] = f16(c.gather(s, c.k_pages, int(n))), f16(c.gather(s, c.v_pages, int(n)))
                    rows.append([kc, vc, 0, int(n), cap])
                self.rings[i] = rows
        self.state = {i: L["state"].copy() for i, L in enumerate(m.layers) if L["kind"] == 0}
        self.x = m.x.copy()

    def step(self):
        orc, m, d = self.orc, self.m, self.m.dims
        H, I, D = d["hidden"], d["inter"], d["head_dim"]
        outs = []
        for i, L in enumerate(m.layers):
            if L["kind"] == 1:
                o = []
                for s, r in enumerate(self.rings[i]):
                    kc, vc, st, ln, cap = r
                    y, r[0], r[1], r[2], r[3] = orc.full_attn_decode(
                        L["q_gate"][s], L["k"][s], L["v"][s], kc, vc, L["q_norm_w"], L["k_norm_w"], d["n_heads"],
                        d["n_kv_heads"], D, d["rot_dim"], ln, d["theta"], d["eps"], 0, True, st, ln, cap)
                    o.append(y.reshape(-1))
                outs.append(np.stack(o))
            else:
                o = []
                for s in range(len(m.lens)):
                    y, self.state[i][s] = orc.deltanet_decode(
                        self.state[i][s], L["dn_q"][s], L["dn_k"][s], L["dn_v"][s], L["dn_a"][s], L["dn_b"][s],
                        L["dn_A"], L["dn_dt_bias"], L["dn_flags"], L["dn_z"][s], L["dn_norm_w"])
                    o.append(y.reshape(-1))
                outs.append(np.stack(o))
            n = np.stack([orc.rmsnorm(xr, L["ffn_norm_w"], d["eps"]) for xr in self.x])
            gu, gl = L["gate_up_w"], L["gate_up_lut"]
            self.x = (self.x + orc.lut6_ffn_batch(n, (gu[:I], gl[:I // 32]), (gu[I:], gl[I // 32:]),
                                                  (L["down_w"], L["down_lut"]), H, I)).astype(np.float32)
        return outs


# ------------------------------------------- serve_hybrid.py CPU attention
def oracle_serve_attention(orc, q_gate16, k16, v16, pos, k_cache, v_cache, cos_row, sin_row,
                           Hq=16, Hkv=4, D=256, rot=64, kv_f16=False):
    """scripts/serve_hybrid.py:85-132 (cpu_attention) as a composition of the
    oracle's cpu_ops functions: widen the fp16 inputs; half-split RoPE of the
    query half of each q_gate row and of k with the given cos/sin row
    (:91-103); k, v into the head-major caches [Hkv][ctx][D] at slot pos
    (:105-106); attention over keys 0..pos (:108-126) -- gqa_attention over
    the token-major view of the caches; the sigmoid gate (:128-130); fp16
    result [1][Hq*D].  Updates k_cache / v_cache (fp32 numpy) in place; with
    kv_f16 the appended rows are stored rounded to fp16 (an fp16 cache)."""
    qg = widen(np.ascontiguousarray(q_gate16, np.uint16)).reshape(Hq, 2 * D)
    k = widen(np.ascontiguousarray(k16, np.uint16)).reshape(Hkv, D)
    v = widen(np.ascontiguousarray(v16, np.uint16)).reshape(Hkv, D)
    qg, k = orc.apply_rope(qg, k, Hq, Hkv, D, 2 * D, D, rot, pos, 1e7, cos_row, sin_row, 1)
    k_cache[:, pos, :] = widen(f16(k)) if kv_f16 else k
    v_cache[:, pos, :] = widen(f16(v)) if kv_f16 else v
    kc = np.ascontiguousarray(k_cache[:, :pos + 1, :].transpose(1, 0, 2))
    vc = np.ascontiguousarray(v_cache[:, :pos + 1, :].transpose(1, 0, 2))
    out = orc.gqa_attention(qg, kc, vc, Hq, Hkv, D, 2 * D, 0, pos + 1, pos + 1)
    out = orc.mul_sigmoid(out, qg[:, D:])
    return f16(out.reshape(1, Hq * D))
