"""GPU parity of the prompt prefill through each layer core from its
projections, against the oracle's per-token decode steps (the reference
prefills by running the decode core once per prompt token: generate.cpp:55-85,
models/llm/qwen3_5.cpp:1164-1217):

* anelm_full_attn_prefill == S x orc_full_attn_decode (q/k RMSNorm, RoPE at
  each position, fp16 ring append, attention over the ring after the append,
  sigmoid gate), over a cached prefix in a wrapped ring, with the ring
  overflowing inside the prompt, without norms / gate, and at the prefill
  workload's size (4096 tokens, 16 q / 4 kv heads) on sampled rows;
* anelm_deltanet_prefill_from_proj == S x orc_deltanet_from_proj (conv ring
  + SiLU + split, l2 norm, gates, recurrence, gated norm): outputs, final
  state, conv ring and its position.
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import assert_close, to_dev, to_host
from workloads import f16, widen

pytestmark = pytest.mark.gpu


def _attn_case(seed, S, Hq, Hkv, D, cap, start, len0):
    rng = np.random.default_rng(seed)
    kc = np.zeros((cap, Hkv, D), np.uint16)
    vc = np.zeros((cap, Hkv, D), np.uint16)
    slots = (start + np.arange(len0)) % cap
    kc[slots] = f16(rng.standard_normal((len0, Hkv, D)))
    vc[slots] = f16(rng.standard_normal((len0, Hkv, D)))
    return dict(q_gate=rng.standard_normal((S, Hq, 2 * D)).astype(np.float32),
                k=rng.standard_normal((S, Hkv, D)).astype(np.float32),
                v=rng.standard_normal((S, Hkv, D)).astype(np.float32),
                kc=kc, vc=vc,
                qw=(1 + 0.02 * rng.standard_normal(D)).astype(np.float32),
                kw=(1 + 0.02 * rng.standard_normal(D)).astype(np.float32))


def _run_prefill(anelm, dev, c, S, Hq, Hkv, D, rot, cap, start, len0, pos0, norms, rope_mode, gate):
    kc, vc = to_dev(c["kc"], dev), to_dev(c["vc"], dev)
    ring = anelm.ops.KVRing(cap, start, len0)
    tab = anelm.ops.rope_table(rot, pos0 + S, 1e7, dev) if rot else None
    out = anelm.ops.full_attn_prefill(to_dev(c["q_gate"], dev), to_dev(c["k"], dev), to_dev(c["v"], dev), kc, vc,
                                      to_dev(c["qw"], dev) if norms else None,
                                      to_dev(c["kw"], dev) if norms else None, ring, Hq, Hkv, D, rot, pos0,
                                      rope_mode=rope_mode, gate=gate, rope_table=tab,
                                      rope_rows=pos0 + S if rot else 0)
    return to_host(out), to_host(kc), to_host(vc), ring.start.value, ring.len.value


@pytest.mark.parametrize("S,Hq,Hkv,D,cap,start,len0,norms,rope_mode,gate", [
    (200, 16, 4, 256, 2048, 1900, 300, True, 0, True),   # 4B heads, cached prefix over the ring's end
    (300, 16, 4, 256, 256, 100, 200, True, 0, True),     # ring overflows inside the prompt (window)
    (97, 4, 2, 128, 1024, 0, 0, False, 1, False),        # empty cache, no norms, half-split, no gate
    (64, 8, 1, 256, 512, 5, 448, True, 0, True),         # G = 8, prompt fills the ring exactly
])
def test_full_attn_prefill_matches_decode_steps(anelm, orc, dev, S, Hq, Hkv, D, cap, start, len0, norms,
                                                rope_mode, gate):
    rot, pos0 = D // 4, len0 + 7
    c = _attn_case(1700 + S + Hq, S, Hq, Hkv, D, cap, start, len0)
    print(f"full_attn_prefill S{S} {Hq}/{Hkv} D{D} cap{cap} len0 {len0}", flush=True)
    got, gk, gv, gs, gl = _run_prefill(anelm, dev, c, S, Hq, Hkv, D, rot, cap, start, len0, pos0, norms,
                                       rope_mode, gate)
    kc, vc, st, ln = c["kc"], c["vc"], start, len0
    for t in range(S):
        want, kc, vc, st, ln = orc.full_attn_decode(c["q_gate"][t], c["k"][t], c["v"][t], kc, vc,
                                                    c["qw"] if norms else None, c["kw"] if norms else None,
                                                    Hq, Hkv, D, rot, pos0 + t, 1e7, 1e-6, rope_mode, gate,
                                                    st, ln, cap)
        assert_close(got[t], want, what=f"row {t}")
    assert (gs, gl) == (st, ln)
    # the ring holds the same keys (fp16 rows of the same normalised, rotated
    # values; a sum-of-squares order may move one rounding)
    assert_close(widen(gk), widen(kc), rel=1e-3, max_abs=2e-3, what="k ring")
    assert np.array_equal(gv, vc), "v ring"


def test_full_attn_prefill_from_projection_rows(anelm, orc, dev):
    """q_gate, k and v read from the first projection's rows [S][q_gate | k |
    v] (proj_stride) give the same results as packed arrays."""
    S, Hq, Hkv, D, cap, rot = 150, 16, 4, 256, 1024, 64
    c = _attn_case(1760, S, Hq, Hkv, D, cap, 10, 37)
    packed = _run_prefill(anelm, dev, c, S, Hq, Hkv, D, rot, cap, 10, 37, 40, True, 0, True)
    proj = np.concatenate([c["q_gate"].reshape(S, -1), c["k"].reshape(S, -1), c["v"].reshape(S, -1)], axis=1)
    kc, vc = to_dev(c["kc"], dev), to_dev(c["vc"], dev)
    ring = anelm.ops.KVRing(cap, 10, 37)
    tab = anelm.ops.rope_table(rot, 40 + S, 1e7, dev)
    out = anelm.ops.full_attn_prefill(None, None, None, kc, vc, to_dev(c["qw"], dev), to_dev(c["kw"], dev), ring,
                                      Hq, Hkv, D, rot, 40, rope_table=tab, rope_rows=40 + S,
                                      proj=to_dev(proj, dev))
    assert np.array_equal(to_host(out), packed[0])
    assert np.array_equal(to_host(kc), packed[1]) and np.array_equal(to_host(vc), packed[2])
    assert (ring.start.value, ring.len.value) == packed[3:]


def test_full_attn_prefill_4096_rows(anelm, orc, dev):
    """The prefill workload's size through the layer core: 4096 prompt tokens,
    16 q / 4 kv heads, D 256, empty 8192-key ring.  Sampled rows against the
    oracle's composition for row t: q/k RMSNorm + RoPE per token, fp16 keys
    0..t, gqa_attention, sigmoid gate."""
    S, Hq, Hkv, D, cap, rot = 4096, 16, 4, 256, 8192, 64
    c = _attn_case(1750, S, Hq, Hkv, D, cap, 0, 0)
    got, gk, gv, gs, gl = _run_prefill(anelm, dev, c, S, Hq, Hkv, D, rot, cap, 0, 0, 0, True, 0, True)
    assert (gs, gl) == (0, S)
    rows = [0, 1, 63, 64, 1000, 2047, 2048, 4095] + list(np.random.default_rng(1751).integers(0, S, 4))
    top = max(int(t) for t in rows)
    # every key normalised and rotated at its own position, fp16 as cached
    kc = np.zeros((cap, Hkv, D), np.uint16)
    zq = np.zeros((1, 2 * D), np.float32)
    for j in range(top + 1):
        kn = orc.rmsnorm(c["k"][j], c["kw"], 1e-6)
        kc[j] = f16(orc.apply_rope(zq, kn, 1, Hkv, D, 2 * D, D, rot, j, 1e7, mode=0)[1])
    vc = np.zeros((cap, Hkv, D), np.uint16)
    vc[:top + 1] = f16(c["v"][:top + 1])
    assert_close(widen(gk[:top + 1]), widen(kc[:top + 1]), rel=1e-3, max_abs=2e-3, what="k ring")
    assert np.array_equal(gv[:S], vc[:S]), "v ring"
    for t in rows:
        t = int(t)
        qn = orc.rmsnorm(c["q_gate"][t, :, :D], c["qw"], 1e-6)
        qg = np.concatenate([qn, c["q_gate"][t, :, D:]], axis=1)
        qr, _ = orc.apply_rope(qg, np.zeros((Hkv, D), np.float32), Hq, Hkv, D, 2 * D, D, rot, t, 1e7, mode=0)
        att = orc.gqa_attention(qr, widen(kc), widen(vc), Hq, Hkv, D, 2 * D, 0, t + 1, cap)
        want = orc.mul_sigmoid(att, c["q_gate"][t, :, D:])
        assert_close(got[t], want, what=f"row {t}")


@pytest.mark.parametrize("S,Hk,Hv,flags,pos0", [
    (100, 16, 32, 5, 2),      # 4B layer: l2 norm + gated norm, conv ring position 2
    (130, 16, 16, 7, 0),      # 0.8B heads, transformers order
    (2, 16, 32, 5, 1),        # fewer tokens than the ring holds
])
def test_deltanet_prefill_from_proj_matches_decode_steps(anelm, orc, dev, S, Hk, Hv, flags, pos0):
    rng = np.random.default_rng(1800 + S + Hv + flags)
    d, K = 128, 4
    qkv = 2 * Hk * d + Hv * d
    St = (0.1 * rng.standard_normal((Hv, d, d))).astype(np.float32)
    conv_w = (0.5 * rng.standard_normal((qkv, K))).astype(np.float32)
    cs = (0.5 * rng.standard_normal((qkv, K - 1))).astype(np.float32)
    A = np.exp(rng.uniform(0, np.log(16), Hv)).astype(np.float32)
    dtb = rng.standard_normal(Hv).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    proj = rng.standard_normal((S, qkv + Hv * d + 2 * Hv)).astype(np.float32)
    Sd, csd = to_dev(St, dev), to_dev(cs, dev)
    pos = ctypes.c_int(pos0)
    print(f"deltanet_prefill_from_proj S{S} {Hk}k/{Hv}v flags {flags}", flush=True)
    y = to_host(anelm.ops.deltanet_prefill_from_proj(Sd, csd, pos, to_dev(proj, dev), to_dev(conv_w, dev),
                                                     to_dev(A, dev), to_dev(dtb, dev), to_dev(nw, dev), Hk,
                                                     flags, K))
    p = pos0
    for t in range(S):
        yw, St, cs, p = orc.deltanet_from_proj(St, cs, p, proj[t], conv_w, A, dtb, nw, Hk, Hv, K, flags)
        assert_close(y[t], yw, what=f"y token {t}")
    assert pos.value == p
    assert_close(to_host(Sd), St, what="state")
    assert np.array_equal(to_host(csd), cs), "conv ring"
