"""Torch-tensor wrappers over the libanelm C ABI.

Every function takes device tensors, launches on torch's current HIP stream
and returns the output tensor(s).  Names and argument meaning follow the
reference's core/cpu_ops.h (rmsnorm, apply_rope_cached, gqa_attention,
ssm_step, ...) and the caller glue in models/llm/qwen3_5.cpp.
"""
from __future__ import annotations

import ctypes

import torch

from . import (ANELM_F16, ANELM_F32, ROPE_INTERLEAVED, call)

_F32 = torch.float32
_F16 = torch.float16


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _s():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need(t, dtype, name):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _floats(vals):
    if vals is None:
        return None
    arr = (ctypes.c_float * len(vals))(*[float(v) for v in vals])
    return ctypes.cast(arr, ctypes.POINTER(ctypes.c_float)), arr


class KVRing:
    """Host-side ring bookkeeping of one KV cache (qwen3_5.h:165-171)."""

    def __init__(self, capacity: int, start: int = 0, length: int = 0):
        self.capacity = capacity
        self.start = ctypes.c_int(start)
        self.len = ctypes.c_int(length)


# ------------------------------------------------------------------ norms
def rmsnorm(x, w, eps=1e-6, out=None):
    """cpu_ops.cpp:24-30 per row of the last dimension."""
    _need(x, _F32, "x")
    dim = x.shape[-1]
    rows = x.numel() // dim
    out = torch.empty_like(x) if out is None else out
    call("anelm_rmsnorm", _p(out), _p(x), _p(w), dim, rows, dim, dim, eps, _s())
    return out


def rmsnorm_gated(x, z, w):
    """cpu_ops.cpp:32-38 per row."""
    dim = x.shape[-1]
    out = torch.empty_like(x)
    call("anelm_rmsnorm_gated", _p(out), _p(x), _p(z), _p(w), dim, x.numel() // dim, _s())
    return out


def l2_normalize_(x):
    """cpu_ops.cpp:82-87 in place per row."""
    dim = x.shape[-1]
    call("anelm_l2_normalize", _p(x), dim, x.numel() // dim, _s())
    return x


def apply_rope_(q, k, n_q_heads, n_kv_heads, head_dim, q_head_stride, k_head_stride, rot_dim,
                pos, theta, rope_mode=ROPE_INTERLEAVED, cos_row=None, sin_row=None):
    """cpu_ops.cpp:40-63 in place; cos_row/sin_row are host sequences or None."""
    c = _floats(cos_row)
    s = _floats(sin_row)
    call("anelm_apply_rope", _p(q), _p(k), n_q_heads, n_kv_heads, head_dim, q_head_stride,
         k_head_stride, rot_dim, pos, theta, c[0] if c else None, s[0] if s else None,
         rope_mode, _s())


def silu_(x):
    call("anelm_silu_inplace", _p(x), x.numel(), _s())
    return x


def mul_sigmoid_(y, z):
    call("anelm_mul_sigmoid_inplace", _p(y), _p(z), y.numel(), _s())
    return y


def softmax_(x):
    n = x.shape[-1]
    call("anelm_softmax", _p(x), n, x.numel() // n, _s())
    return x


def matvec(W, x):
    out = torch.empty(W.shape[0], device=x.device, dtype=_F32)
    call("anelm_matvec", _p(out), _p(W), _p(x), W.shape[0], W.shape[1], _s())
    return out


def conv1d_update(conv_state, state_pos: ctypes.c_int, x, w, kernel_size):
    channels = x.numel()
    y = torch.empty_like(x)
    call("anelm_conv1d_update", _p(y), _p(conv_state), ctypes.byref(state_pos), _p(x), _p(w),
         channels, kernel_size, _s())
    return y


# -------------------------------------------------------------- attention
def gqa_attention(q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, q_head_stride,
                  cache_start, cache_len, cache_capacity, out=None):
    """cpu_ops.cpp:148-204; caches fp32 or fp16 [cap][Hkv][D]."""
    kv = ANELM_F16 if k_cache.dtype == _F16 else ANELM_F32
    out = torch.empty(n_heads, head_dim, device=q.device, dtype=_F32) if out is None else out
    call("anelm_gqa_attention", _p(out), _p(q), _p(k_cache), _p(v_cache), kv, n_heads,
         n_kv_heads, head_dim, q_head_stride, cache_start, cache_len, cache_capacity, _s())
    return out


def full_attn_decode(q_gate, k, v, k_cache, v_cache, q_norm_w, k_norm_w, ring: KVRing,
                     n_heads, n_kv_heads, head_dim, rot_dim, pos, theta=1e7, eps=1e-6,
                     rope_mode=ROPE_INTERLEAVED, gate=True, cos_row=None, sin_row=None,
                     out=None):
    """qwen3_5.cpp:944-1002 fused: norms, RoPE, fp16 ring append, attention, gate."""
    _need(k_cache, _F16, "k_cache")
    out = torch.empty(n_heads, head_dim, device=q_gate.device, dtype=_F32) if out is None else out
    c = _floats(cos_row)
    s = _floats(sin_row)
    call("anelm_full_attn_decode", _p(out), _p(q_gate), _p(k), _p(v), _p(k_cache), _p(v_cache),
         _p(q_norm_w), _p(k_norm_w), n_heads, n_kv_heads, head_dim, rot_dim, pos, theta, eps,
         rope_mode, 1 if gate else 0, c[0] if c else None, s[0] if s else None,
         ctypes.byref(ring.start), ctypes.byref(ring.len), ring.capacity, _s())
    return out


def full_attn_decode_kv(q_gate, k, v, k_cache, v_cache, layout, q_norm_w, k_norm_w, ring: KVRing,
                        n_heads, n_kv_heads, head_dim, rot_dim, pos, theta=1e7, eps=1e-6,
                        rope_mode=ROPE_INTERLEAVED, gate=True, cos_row=None, sin_row=None, out=None):
    """full_attn_decode over an fp16 or fp32 cache, token-major (layout 0) or
    head-major [Hkv][cap][D] (layout 1)."""
    kv_dtype = ANELM_F16 if k_cache.dtype == _F16 else ANELM_F32
    out = torch.empty(n_heads, head_dim, device=q_gate.device, dtype=_F32) if out is None else out
    c = _floats(cos_row)
    s = _floats(sin_row)
    call("anelm_full_attn_decode_kv", _p(out), _p(q_gate), _p(k), _p(v), _p(k_cache), _p(v_cache), kv_dtype,
         layout, _p(q_norm_w), _p(k_norm_w), n_heads, n_kv_heads, head_dim, rot_dim, pos, theta, eps,
         rope_mode, 1 if gate else 0, c[0] if c else None, s[0] if s else None,
         ctypes.byref(ring.start), ctypes.byref(ring.len), ring.capacity, _s())
    return out


def attn_decode_paged(q, k_pages, v_pages, page_table, seq_lens, max_seq_len, n_heads,
                      n_kv_heads, head_dim, page_size, q_head_stride=None, out=None):
    n_seqs = seq_lens.numel()
    max_pages = page_table.shape[-1]
    q_head_stride = head_dim if q_head_stride is None else q_head_stride
    out = (torch.empty(n_seqs, n_heads, head_dim, device=q.device, dtype=_F32)
           if out is None else out)
    n_pages = k_pages.shape[0]
    call("anelm_attn_decode_paged", _p(out), _p(q), q_head_stride, _p(k_pages), _p(v_pages),
         _p(page_table), _p(seq_lens), n_seqs, max_pages, page_size, n_pages, max_seq_len,
         n_heads, n_kv_heads, head_dim, _s())
    return out


def rope_table(rot_dim, n_pos, theta, device):
    """RoPE rows 0..n_pos-1 on the device: [n_pos][rot_dim] = cos pairs, sin pairs."""
    t = torch.empty(n_pos, rot_dim, device=device, dtype=_F32)
    call("anelm_rope_table", _p(t), rot_dim, n_pos, theta)
    return t


def attn_decode_paged_step(q_gate, k, v, k_pages, v_pages, page_table, seq_lens, q_norm_w, k_norm_w,
                           max_seq_len, n_heads, n_kv_heads, head_dim, page_size, rot_dim, theta=1e7,
                           eps=1e-6, rope_mode=ROPE_INTERLEAVED, gate=True, positions=None, rope_tab=None,
                           out=None):
    """qwen3_5.cpp:944-1002 per sequence over paged fp16 caches: norms, RoPE,
    page append of the new key (key seq_lens[s]), attention over
    seq_lens[s] + 1 keys, gate.  seq_lens is not advanced."""
    n_seqs = seq_lens.numel()
    out = (torch.empty(n_seqs, n_heads, head_dim, device=q_gate.device, dtype=_F32)
           if out is None else out)
    call("anelm_attn_decode_paged_step", _p(out), _p(q_gate), _p(k), _p(v), _p(k_pages), _p(v_pages),
         _p(page_table), _p(seq_lens), _p(positions), _p(q_norm_w), _p(k_norm_w), _p(rope_tab),
         0 if rope_tab is None else rope_tab.shape[0], n_seqs, page_table.shape[-1], page_size,
         k_pages.shape[0], max_seq_len, n_heads, n_kv_heads, head_dim, rot_dim, theta, eps, rope_mode,
         1 if gate else 0, _s())
    return out


def attn_prefill(q, k, v, out_dtype=_F32):
    """Causal GQA prefill; q [S][Hq][D], k/v [S][Hkv][D] fp16."""
    S, Hq, D = q.shape
    Hkv = k.shape[1]
    out = torch.empty(S, Hq, D, device=q.device, dtype=out_dtype)
    call("anelm_attn_prefill", _p(out), ANELM_F16 if out_dtype == _F16 else ANELM_F32, _p(q),
         _p(k), _p(v), S, Hq, Hkv, D, _s())
    return out


def full_attn_prefill(q_gate, k, v, k_cache, v_cache, q_norm_w, k_norm_w, ring: KVRing, n_heads,
                      n_kv_heads, head_dim, rot_dim, pos0, theta=1e7, eps=1e-6, rope_mode=ROPE_INTERLEAVED,
                      gate=True, rope_table=None, rope_rows=0, proj=None):
    """S tokens of qwen3_5.cpp:944-1002 over the fp16 ring in one call;
    q_gate [S][Hq][2D], k/v [S][Hkv][D] -- or proj [S][q_gate | k | v] (the
    first projection's rows; q_gate, k, v ignored); returns out [S][Hq][D]."""
    _need(k_cache, _F16, "k_cache")
    stride = 0
    if proj is not None:
        S, stride = proj.shape
        base = proj.data_ptr()
        q_gate, k = proj, None
        qp = ctypes.c_void_p(base)
        kp = ctypes.c_void_p(base + 4 * n_heads * 2 * head_dim)
        vp = ctypes.c_void_p(base + 4 * (n_heads * 2 * head_dim + n_kv_heads * head_dim))
    else:
        S = q_gate.shape[0]
        qp, kp, vp = _p(q_gate), _p(k), _p(v)
    out = torch.empty(S, n_heads, head_dim, device=q_gate.device, dtype=_F32)
    call("anelm_full_attn_prefill", _p(out), qp, kp, vp, stride, _p(k_cache), _p(v_cache),
         _p(q_norm_w), _p(k_norm_w), S, n_heads, n_kv_heads, head_dim, rot_dim, pos0, theta, eps, rope_mode,
         1 if gate else 0, _p(rope_table), rope_rows, ctypes.byref(ring.start), ctypes.byref(ring.len),
         ring.capacity, _s())
    return out


# --------------------------------------------------------------- DeltaNet
def ssm_step(state, q, k, v, decay, beta, flags=0):
    """cpu_ops.cpp:131-146 on one head; state [dk][dv] updated in place."""
    y = torch.empty(state.shape[1], device=state.device, dtype=_F32)
    call("anelm_ssm_step", _p(y), _p(state), _p(q), _p(k), _p(v), decay, beta, state.shape[0],
         state.shape[1], flags, _s())
    return y


def deltanet_decode(state, q, k, v, a, b, A, dt_bias, flags, z=None, norm_w=None, out=None):
    """qwen3_5.cpp:879-908; state [Hv][dk][dv] updated in place."""
    Hv, dk, dv = state.shape
    Hk = q.shape[0]
    out = torch.empty(Hv, dv, device=state.device, dtype=_F32) if out is None else out
    call("anelm_deltanet_decode", _p(out), _p(state), _p(q), _p(k), _p(v), _p(a), _p(b), _p(A),
         _p(dt_bias), _p(z), _p(norm_w), Hk, Hv, dk, dv, flags, _s())
    return out


def deltanet_decode_batched(state, q, k, v, a, b, A, dt_bias, flags, z, norm_w, n_seqs, out=None):
    """n_seqs sequences' DeltaNet steps in one launch; state [n_seqs*Hv][dk][dv],
    q,k [n_seqs*Hk][dk], v,z [n_seqs*Hv][dv], a,b [n_seqs*Hv]; A, dt_bias [Hv]
    and norm_w [dv] are the layer's, shared by the sequences."""
    Hv = A.numel()
    Hk = q.numel() // (n_seqs * q.shape[-1])
    out = torch.empty(n_seqs * Hv, v.shape[-1], device=v.device, dtype=_F32) if out is None else out
    call("anelm_deltanet_decode_batched", _p(out), _p(state), _p(q), _p(k), _p(v), _p(a), _p(b), _p(A),
         _p(dt_bias), _p(z), _p(norm_w), n_seqs, Hk, Hv, q.shape[-1], v.shape[-1], flags, _s())
    return out


def deltanet_decode_from_proj(state, conv_state, conv_pos, proj, conv_w, A, dt_bias, norm_w, Hk, flags,
                              conv_kernel=4, out=None):
    """qwen3_5.cpp:849-908 from the norm-fused first projection
    proj = [q|k|v mixed | z | a | b]; conv_state [qkv][K-1] and state
    [Hv][dk][dv] are updated in place; conv_pos is a ctypes.c_int advanced
    here."""
    Hv, dk, dv = state.shape
    out = torch.empty(Hv, dv, device=state.device, dtype=_F32) if out is None else out
    call("anelm_deltanet_decode_from_proj", _p(out), _p(state), _p(conv_state), ctypes.byref(conv_pos),
         _p(proj), _p(conv_w), _p(A), _p(dt_bias), _p(norm_w), Hk, Hv, dk, dv, conv_kernel, flags, _s())
    return out


def deltanet_prefill_from_proj(state, conv_state, conv_pos: ctypes.c_int, proj, conv_w, A, dt_bias, norm_w,
                               Hk, flags, conv_kernel=4):
    """S tokens of qwen3_5.cpp:849-908 from the projections; proj [S][proj_dim]."""
    Hv, dk, dv = state.shape
    S = proj.shape[0]
    y = torch.empty(S, Hv, dv, device=state.device, dtype=_F32)
    call("anelm_deltanet_prefill_from_proj", _p(y), _p(state), _p(conv_state), ctypes.byref(conv_pos),
         _p(proj), _p(conv_w), _p(A), _p(dt_bias), _p(norm_w), S, Hk, Hv, dk, dv, conv_kernel, flags, _s())
    return y


def deltanet_prefill(state, q, k, v, a, b, A, dt_bias, flags, chunk=64):
    """Chunked prefill; q,k [S][Hk][dk], v [S][Hv][dv], a,b [S][Hv]."""
    S, Hk, dk = q.shape
    Hv, _, dv = state.shape
    y = torch.empty(S, Hv, dv, device=state.device, dtype=_F32)
    call("anelm_deltanet_prefill", _p(y), _p(state), _p(q), _p(k), _p(v), _p(a), _p(b), _p(A),
         _p(dt_bias), S, Hk, Hv, dk, dv, chunk, flags, _s())
    return y


# ------------------------------------------------------------------- LUT6
def lut6_unpack(packed, n):
    idx = torch.empty(n, device=packed.device, dtype=torch.uint8)
    call("anelm_lut6_unpack", _p(idx), _p(packed), n, _s())
    return idx


def lut6_proj(w, lut, x, out_dim, in_dim, norm_w=None, eps=1e-6, y=None, accumulate=False):
    """y = W rmsnorm(x, norm_w) (norm_w None: W x); with accumulate, y += W n."""
    y = torch.empty(out_dim, device=x.device, dtype=_F32) if y is None else y
    call("anelm_lut6_proj", _p(y), _p(w), _p(lut), _p(x), _p(norm_w), eps, out_dim, in_dim,
         1 if accumulate else 0, _s())
    return y


def lut6_gemv(w, lut, x, out_dim, in_dim, out=None):
    out = torch.empty(out_dim, device=x.device, dtype=_F32) if out is None else out
    call("anelm_lut6_gemv", _p(out), _p(w), _p(lut), _p(x), out_dim, in_dim, _s())
    return out


def lut6_ffn_(x, gu_scratch, norm_w, eps, gate, up, down, hidden, inter):
    """x += down(silu(gate n) * (up n)), n = rmsnorm(x, norm_w); gate/up/down = (w, lut);
    gu_scratch holds 2*inter floats."""
    if gu_scratch.numel() < 2 * inter:
        raise ValueError("gu_scratch needs 2*inter floats")
    call("anelm_lut6_ffn", _p(x), _p(gu_scratch), _p(norm_w), eps, _p(gate[0]), _p(gate[1]),
         _p(up[0]), _p(up[1]), _p(down[0]), _p(down[1]), hidden, inter, _s())
    return x


def lut6_gate_up(x, norm_w, eps, gate, up, hidden, inter):
    """(gate n, up n), n = rmsnorm(x, norm_w) (x when norm_w is None)."""
    g = torch.empty(inter, device=x.device, dtype=_F32)
    u = torch.empty(inter, device=x.device, dtype=_F32)
    call("anelm_lut6_gate_up", _p(g), _p(u), _p(x), _p(norm_w), eps, _p(gate[0]), _p(gate[1]),
         _p(up[0]), _p(up[1]), hidden, inter, _s())
    return g, u


def lut6_gemm(w, lut, x, out_dim, in_dim, out=None, accumulate=False):
    """y[b] = W x[b] (or y[b] += W x[b]) for a batch x [batch][in_dim]
    (weights dequantised once per 32 inputs)."""
    batch = x.shape[0]
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs out")
        out = torch.empty(batch, out_dim, device=x.device, dtype=_F32)
    call("anelm_lut6_gemm", _p(out), _p(w), _p(lut), _p(x), batch, out_dim, in_dim, 1 if accumulate else 0, _s())
    return out


def swiglu(g, u, out=None):
    """silu(g) * u elementwise."""
    out = torch.empty_like(g) if out is None else out
    call("anelm_swiglu", _p(out), _p(g), _p(u), g.numel(), _s())
    return out


def swiglu_rows(gu, n, out=None):
    """h[r] = silu(gu[r][:n]) * gu[r][n:2n] for the stacked gate / up output gu [rows][2n]."""
    rows = gu.numel() // (2 * n)
    out = out if out is not None else torch.empty(rows, n, device=gu.device)
    call("anelm_swiglu_rows", _p(out), _p(gu), rows, n, _s())
    return out


def lut6_topk(w, lut, x, out_dim, in_dim, k):
    batch = x.shape[0] if x.dim() == 2 else 1
    idx = torch.empty(batch, k, device=x.device, dtype=torch.int32)
    val = torch.empty(batch, k, device=x.device, dtype=_F32)
    call("anelm_lut6_topk", _p(idx), _p(val), _p(w), _p(lut), _p(x), batch, out_dim, in_dim, k,
         _s())
    return idx, val


# --------------------------------------------------------------- sampling
def sample_token(logits, recent, temperature, repetition_penalty=1.2, repetition_context_size=256,
                 frequency_penalty=0.1, r=0.5, out=None):
    """core/sampling.cpp:11-66 on the device; recent is a device int32 tensor
    (or None), r the uniform draw.  Returns a device int32 [1] tensor."""
    out = torch.empty(1, device=logits.device, dtype=torch.int32) if out is None else out
    n = 0 if recent is None else recent.numel()
    call("anelm_sample_token", _p(out), _p(logits), logits.numel(), _p(recent), n, temperature,
         repetition_penalty, repetition_context_size, frequency_penalty, r, _s())
    return out
