"""numpy binding of liboracle.so, the CPU restatement of ANE-LM's cpu_ops path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the oracle.  The product library never uses
it.  Every wrapper names the C function (and through it the reference
file:line) it calls.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_long
_F = ctypes.c_float
_IP = ctypes.POINTER(ctypes.c_int)

_SIGS = {
    "orc_f16_to_f32_array": (None, [_P, _P, _L]),
    "orc_f32_to_f16_array": (None, [_P, _P, _L]),
    "orc_silu_vec_inplace": (None, [_P, _I]),
    "orc_mul_sigmoid_inplace": (None, [_P, _P, _I]),
    "orc_rmsnorm": (None, [_P, _P, _P, _I, _F]),
    "orc_rmsnorm_gated": (None, [_P, _P, _P, _P, _I]),
    "orc_apply_rope": (None, [_P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P, _I]),
    "orc_rope_table": (None, [_P, _P, _I, _I, _F]),
    "orc_softmax": (None, [_P, _I]),
    "orc_matvec": (None, [_P, _P, _P, _I, _I]),
    "orc_l2_normalize": (None, [_P, _I]),
    "orc_conv1d_update": (None, [_P, _P, _IP, _P, _P, _I, _I]),
    "orc_ssm_step": (None, [_P, _P, _P, _P, _P, _F, _F, _I, _I, _I]),
    "orc_gqa_attention": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I]),
    "orc_full_attn_decode": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F,
                                    _I, _I, _IP, _IP, _I]),
    "orc_deltanet_decode": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "orc_prefill_attention": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "orc_deltanet_prefill": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "orc_lut6_pack": (None, [_P, _P, _L]),
    "orc_lut6_unpack": (None, [_P, _P, _L]),
    "orc_lut6_dequant_row": (None, [_P, _P, _P, _I]),
    "orc_lut6_matvec": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "orc_lut6_matvec_batch": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "orc_lut6_ffn_batch": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "orc_lut6_ffn": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P]),
    "orc_topk": (None, [_P, _P, _P, _L, _I]),
    "orc_argmax": (_I, [_P, _I]),
    "orc_deltanet_from_proj": (None, [_P, _P, _P, _IP, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "orc_sample_token": (_I, [_P, _P, _I, _P, _I, _F, _F, _I, _F, _F]),
}

_lib = None
TIMING_LIB_PATH = os.path.join(_HERE, "liboracle_timing.so")


def use_timing_build() -> None:
    """Switches this module to liboracle_timing.so: the same C sources built
    with vectorised (reassociated) reductions, for the CPU-baseline timing in
    bench.py only -- never for checking results."""
    global _lib, LIB_PATH
    LIB_PATH = TIMING_LIB_PATH
    _lib = None
    lib()


def build() -> None:
    """Compiles liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-B", "-C", _HERE, "liboracle.so"], check=True,
                   stdout=subprocess.DEVNULL)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            if LIB_PATH == TIMING_LIB_PATH:
                subprocess.run(["make", "-B", "-C", _HERE, "liboracle_timing.so"], check=True,
                               stdout=subprocess.DEVNULL)
            else:
                build()
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- fp16
def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_array(_p(out), _p(h), h.size)
    return out


def f32_to_f16(x):
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(out), _p(x), x.size)
    return out


# ------------------------------------------------------------- cpu_ops
def silu(x):
    y = _f32(x).copy()
    lib().orc_silu_vec_inplace(_p(y), y.size)
    return y


def mul_sigmoid(y, z):
    y = _f32(y).copy()
    z = _f32(z)
    lib().orc_mul_sigmoid_inplace(_p(y), _p(z), y.size)
    return y


def rmsnorm(x, w, eps=1e-6):
    """orc_rmsnorm per row of the last axis."""
    x = _f32(x)
    w = _f32(w)
    out = np.empty_like(x)
    d = x.shape[-1]
    for r in range(x.size // d):
        lib().orc_rmsnorm(_p(out.reshape(-1, d)[r:r + 1]), _p(x.reshape(-1, d)[r:r + 1]), _p(w), d, eps)
    return out


def rmsnorm_gated(x, z, w):
    x = _f32(x)
    z = _f32(z)
    w = _f32(w)
    out = np.empty_like(x)
    d = x.shape[-1]
    xr, zr, orr = x.reshape(-1, d), z.reshape(-1, d), out.reshape(-1, d)
    for r in range(xr.shape[0]):
        lib().orc_rmsnorm_gated(_p(orr[r:r + 1]), _p(xr[r:r + 1]), _p(zr[r:r + 1]), _p(w), d)
    return out


def apply_rope(q, k, n_q_heads, n_kv_heads, head_dim, q_head_stride, k_head_stride, rot_dim, pos,
               theta, cos_row=None, sin_row=None, mode=0):
    """orc_apply_rope on copies; returns (q, k)."""
    q = _f32(q).copy()
    k = _f32(k).copy()
    c = None if cos_row is None else _f32(cos_row)
    s = None if sin_row is None else _f32(sin_row)
    lib().orc_apply_rope(_p(q), _p(k), n_q_heads, n_kv_heads, head_dim, q_head_stride,
                         k_head_stride, rot_dim, pos, theta, _p(c), _p(s), mode)
    return q, k


def rope_table(max_pos, rot_dim, theta):
    c = np.empty((max_pos, rot_dim // 2), np.float32)
    s = np.empty((max_pos, rot_dim // 2), np.float32)
    lib().orc_rope_table(_p(c), _p(s), max_pos, rot_dim, theta)
    return c, s


def softmax(x):
    x = _f32(x).copy()
    lib().orc_softmax(_p(x), x.size)
    return x


def matvec(W, x):
    W = _f32(W)
    x = _f32(x)
    y = np.empty(W.shape[0], np.float32)
    lib().orc_matvec(_p(y), _p(W), _p(x), W.shape[0], W.shape[1])
    return y


def l2_normalize(x):
    x = _f32(x).copy()
    lib().orc_l2_normalize(_p(x), x.size)
    return x


def conv1d_update(conv_state, state_pos, x, w, kernel_size):
    """Returns (y, new_state, new_pos)."""
    st = _f32(conv_state).copy()
    x = _f32(x)
    w = _f32(w)
    y = np.empty_like(x)
    pos = ctypes.c_int(state_pos)
    lib().orc_conv1d_update(_p(y), _p(st), ctypes.byref(pos), _p(x), _p(w), x.size, kernel_size)
    return y, st, pos.value


def ssm_step(state, q, k, v, decay, beta, order=0):
    """Returns (y, new_state)."""
    S = _f32(state).copy()
    dk, dv = S.shape
    y = np.empty(dv, np.float32)
    lib().orc_ssm_step(_p(y), _p(S), _p(_f32(q)), _p(_f32(k)), _p(_f32(v)), decay, beta, dk, dv,
                       order)
    return y, S


def gqa_attention(q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, q_head_stride, cache_start,
                  cache_len, cache_capacity):
    out = np.empty((n_heads, head_dim), np.float32)
    lib().orc_gqa_attention(_p(out), _p(_f32(q)), _p(_f32(k_cache)), _p(_f32(v_cache)), n_heads,
                            n_kv_heads, head_dim, q_head_stride, cache_start, cache_len,
                            cache_capacity)
    return out


# --------------------------------------------------------- compositions
def full_attn_decode(q_gate, k, v, k_cache, v_cache, q_norm_w, k_norm_w, n_heads, n_kv_heads,
                     head_dim, rot_dim, pos, theta, eps, rope_mode, gate, cache_start, cache_len,
                     cache_capacity):
    """orc_full_attn_decode on copies of the caches.
    Returns (out, k_cache, v_cache, start, len)."""
    qg = _f32(q_gate).copy()
    kk = _f32(k).copy()
    kc = np.ascontiguousarray(k_cache, np.uint16).copy()
    vc = np.ascontiguousarray(v_cache, np.uint16).copy()
    st = ctypes.c_int(cache_start)
    ln = ctypes.c_int(cache_len)
    out = np.empty((n_heads, head_dim), np.float32)
    qn = None if q_norm_w is None else _f32(q_norm_w)
    kn = None if k_norm_w is None else _f32(k_norm_w)
    lib().orc_full_attn_decode(_p(out), _p(qg), _p(kk), _p(_f32(v)), _p(kc), _p(vc),
                               None if qn is None else _p(qn), None if kn is None else _p(kn),
                               n_heads, n_kv_heads,
                               head_dim, rot_dim, pos, theta, eps, rope_mode, 1 if gate else 0,
                               ctypes.byref(st), ctypes.byref(ln), cache_capacity)
    return out, kc, vc, st.value, ln.value


def deltanet_decode(state, q, k, v, a, b, A, dt_bias, flags, z=None, norm_w=None):
    """Returns (y, new_state)."""
    S = _f32(state).copy()
    Hv, dk, dv = S.shape
    qq = _f32(q).copy()
    kk = _f32(k).copy()
    Hk = qq.shape[0]
    y = np.empty((Hv, dv), np.float32)
    zz = None if z is None else _f32(z)
    nw = None if norm_w is None else _f32(norm_w)
    lib().orc_deltanet_decode(_p(y), _p(S), _p(qq), _p(kk), _p(_f32(v)), _p(_f32(a)), _p(_f32(b)),
                              _p(_f32(A)), _p(_f32(dt_bias)), _p(zz), _p(nw), Hk, Hv, dk, dv, flags)
    return y, S


def prefill_attention(q16, k16, v16, row_begin=0, row_end=None):
    """orc_prefill_attention; inputs fp16 bit patterns [S][H][D]."""
    q16 = np.ascontiguousarray(q16, np.uint16)
    k16 = np.ascontiguousarray(k16, np.uint16)
    v16 = np.ascontiguousarray(v16, np.uint16)
    S, Hq, D = q16.shape
    Hkv = k16.shape[1]
    row_end = S if row_end is None else row_end
    out = np.empty((row_end - row_begin, Hq, D), np.float32)
    lib().orc_prefill_attention(_p(out), _p(q16), _p(k16), _p(v16), S, Hq, Hkv, D, row_begin,
                                row_end)
    return out


def deltanet_prefill(state, q, k, v, a, b, A, dt_bias, flags):
    """Returns (y [S][Hv][dv], new_state)."""
    St = _f32(state).copy()
    Hv, dk, dv = St.shape
    qq = _f32(q).copy()
    kk = _f32(k).copy()
    S, Hk, _ = qq.shape
    y = np.empty((S, Hv, dv), np.float32)
    lib().orc_deltanet_prefill(_p(y), _p(St), _p(qq), _p(kk), _p(_f32(v)), _p(_f32(a)),
                               _p(_f32(b)), _p(_f32(A)), _p(_f32(dt_bias)), S, Hk, Hv, dk, dv,
                               flags)
    return y, St


# ---------------------------------------------------------------- LUT6
def lut6_pack(idx):
    idx = np.ascontiguousarray(idx, np.uint8)
    out = np.empty(idx.size * 3 // 4, np.uint8)
    lib().orc_lut6_pack(_p(out), _p(idx), idx.size)
    return out


def lut6_unpack(packed, n):
    packed = np.ascontiguousarray(packed, np.uint8)
    out = np.empty(n, np.uint8)
    lib().orc_lut6_unpack(_p(out), _p(packed), n)
    return out


def lut6_matvec(w, lut, x, out_dim, in_dim, row_begin=0, row_end=None):
    row_end = out_dim if row_end is None else row_end
    y = np.empty(row_end - row_begin, np.float32)
    lib().orc_lut6_matvec(_p(y), _p(np.ascontiguousarray(w, np.uint8)),
                          _p(np.ascontiguousarray(lut, np.uint16)), _p(_f32(x)), out_dim, in_dim,
                          row_begin, row_end)
    return y


def lut6_matvec_batch(w, lut, x, out_dim, in_dim):
    """y[b] = lut6_matvec(x[b]) for x [batch][in_dim], bit-identical per input."""
    x = _f32(x).reshape(-1, in_dim)
    y = np.empty((x.shape[0], out_dim), np.float32)
    lib().orc_lut6_matvec_batch(_p(y), _p(np.ascontiguousarray(w, np.uint8)),
                                _p(np.ascontiguousarray(lut, np.uint16)), _p(x), x.shape[0], out_dim, in_dim)
    return y


def lut6_ffn_batch(x, gate, up, down, hidden, inter):
    """lut6_ffn per row of x [batch][hidden], bit-identical per row."""
    x = _f32(x).reshape(-1, hidden)
    y = np.empty_like(x)
    scratch = np.empty(3 * x.shape[0] * inter, np.float32)
    c = np.ascontiguousarray
    lib().orc_lut6_ffn_batch(_p(y), _p(c(gate[0], np.uint8)), _p(c(gate[1], np.uint16)),
                             _p(c(up[0], np.uint8)), _p(c(up[1], np.uint16)),
                             _p(c(down[0], np.uint8)), _p(c(down[1], np.uint16)), _p(x), x.shape[0],
                             hidden, inter, _p(scratch))
    return y


def lut6_ffn(x, gate, up, down, hidden, inter):
    """down(silu(gate x) * (up x)); gate/up/down = (packed, lut)."""
    y = np.empty(hidden, np.float32)
    scratch = np.empty(2 * inter, np.float32)
    c = np.ascontiguousarray
    lib().orc_lut6_ffn(_p(y), _p(c(gate[0], np.uint8)), _p(c(gate[1], np.uint16)),
                       _p(c(up[0], np.uint8)), _p(c(up[1], np.uint16)),
                       _p(c(down[0], np.uint8)), _p(c(down[1], np.uint16)), _p(_f32(x)), hidden,
                       inter, _p(scratch))
    return y


def topk(logits, k):
    logits = _f32(logits)
    idx = np.empty(k, np.int32)
    val = np.empty(k, np.float32)
    lib().orc_topk(_p(idx), _p(val), _p(logits), logits.size, k)
    return idx, val


def argmax(logits):
    logits = _f32(logits)
    return int(lib().orc_argmax(_p(logits), logits.size))


def deltanet_from_proj(state, conv_state, conv_pos, proj, conv_w, A, dt_bias, norm_w, Hk, Hv,
                       kernel_size, flags):
    """orc_deltanet_from_proj (qwen3_5.cpp:849-908) on copies.
    Returns (y, state, conv_state, conv_pos)."""
    S = _f32(state).copy()
    cs = _f32(conv_state).copy()
    dk, dv = S.shape[1], S.shape[2]
    y = np.empty((Hv, dv), np.float32)
    pos = ctypes.c_int(conv_pos)
    nw = None if norm_w is None else _f32(norm_w)
    lib().orc_deltanet_from_proj(_p(y), _p(S), _p(cs), ctypes.byref(pos), _p(_f32(proj)), _p(_f32(conv_w)),
                                 _p(_f32(A)), _p(_f32(dt_bias)), _p(nw), Hk, Hv, dk, dv, kernel_size,
                                 flags)
    return y, S, cs, pos.value


def sample_token(logits, recent, temperature, repetition_penalty, repetition_context_size,
                 frequency_penalty, r):
    """orc_sample_token (core/sampling.cpp:11-66, draw r given).
    Returns (token, adjusted values)."""
    lg = _f32(logits)
    adj = np.empty_like(lg)
    rec = np.ascontiguousarray(recent, np.int32)
    tok = lib().orc_sample_token(_p(adj), _p(lg), lg.size, _p(rec) if rec.size else None, rec.size,
                                 temperature, repetition_penalty, repetition_context_size,
                                 frequency_penalty, r)
    return int(tok), adj
