"""Drop-in for the CPU attention of scripts/serve_hybrid.py on the GPU.

``cpu_attention(q_gate_fp16, k_fp16, v_fp16, pos, kv_caches, layer_idx)`` keeps
the reference function's name, arguments and result (scripts/serve_hybrid.py:
85-132): fp16 ``q_gate`` [16][512] (query | gate per head), ``k``, ``v``
[4][256] from the fused ANE projection; ``kv_caches[layer_idx]`` = (k_cache,
v_cache), head-major [NUM_KV_HEADS][CONTEXT][HEAD_DIM]; half-split RoPE on the
first 64 dims at ``pos`` from the module's cos/sin table; k and v written at
slot ``pos``; attention over keys 0..pos; sigmoid gate; returns fp16
[1][ATTN_DIM].  The work is ONE call of ``anelm_full_attn_decode_kv`` (no q/k
norm, head-major cache, ring starting at slot 0).

The caches live in device memory (``make_kv_caches``; fp32 like the
reference's, or fp16 to halve the bytes read per step).  Inputs may be host
numpy arrays, as the ANE returns them (copied to the device and the result
back), or device tensors (the result stays on the device).
"""
from __future__ import annotations

import numpy as np
import torch

from . import KV_HEAD_MAJOR, ROPE_HALF_SPLIT, ops

# Model constants of the reference server (scripts/serve_hybrid.py:33-40).
NUM_HEADS = 16
NUM_KV_HEADS = 4
HEAD_DIM = 256
ROPE_DIM = 64
ATTN_DIM = NUM_HEADS * HEAD_DIM
CONTEXT = 4096
ROPE_THETA = 10000000.0

# cos/sin table of the reference server (scripts/serve_hybrid.py:50-55), built
# the same way so the rotation angles are the same fp32 values.
_inv_freq = 1.0 / (ROPE_THETA ** (np.arange(0, ROPE_DIM, 2, dtype=np.float32) / ROPE_DIM))
_freqs = np.outer(np.arange(CONTEXT, dtype=np.float32), _inv_freq)
ROPE_COS = np.cos(_freqs).astype(np.float32)
ROPE_SIN = np.sin(_freqs).astype(np.float32)


def make_kv_caches(n_layers, device="cuda", dtype=torch.float32):
    """Zeroed head-major caches, one (k, v) pair per attention layer
    (scripts/serve_hybrid.py:232-235)."""
    shape = (NUM_KV_HEADS, CONTEXT, HEAD_DIM)
    return [(torch.zeros(shape, device=device, dtype=dtype), torch.zeros(shape, device=device, dtype=dtype))
            for _ in range(n_layers)]


def cpu_attention(q_gate_fp16, k_fp16, v_fp16, pos, kv_caches, layer_idx):
    k_cache, v_cache = kv_caches[layer_idx]
    if not (0 <= pos < CONTEXT):
        raise ValueError(f"pos {pos} outside the {CONTEXT}-slot cache")
    host = isinstance(q_gate_fp16, np.ndarray)
    dev = k_cache.device

    def f32(a, shape):
        t = torch.from_numpy(np.ascontiguousarray(a)) if host else a
        return t.to(device=dev, dtype=torch.float32).reshape(shape).contiguous()

    q_gate = f32(q_gate_fp16, (NUM_HEADS, 2 * HEAD_DIM))
    k = f32(k_fp16, (NUM_KV_HEADS, HEAD_DIM))
    v = f32(v_fp16, (NUM_KV_HEADS, HEAD_DIM))
    ring = ops.KVRing(CONTEXT, 0, pos)
    out = ops.full_attn_decode_kv(q_gate, k, v, k_cache, v_cache, KV_HEAD_MAJOR, None, None, ring, NUM_HEADS,
                                  NUM_KV_HEADS, HEAD_DIM, ROPE_DIM, pos, ROPE_THETA,
                                  rope_mode=ROPE_HALF_SPLIT, gate=True,
                                  cos_row=ROPE_COS[pos], sin_row=ROPE_SIN[pos])
    out = out.to(torch.float16).reshape(1, ATTN_DIM)
    return out.cpu().numpy() if host else out
