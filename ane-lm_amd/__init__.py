"""ane-lm_amd: MI355X (gfx950) HIP implementation of ANE-LM's core/cpu_ops hot path.

The product is the C-ABI shared library ``libanelm.so`` (declared in
``include/anelm.h`` and ``include/anelm_cpu_ops.h``).  This package binds it
with ctypes -- the same mechanism the reference's Python server uses for its
CPU attention (scripts/serve_hybrid.py:57-82) -- and offers thin wrappers that
take torch device tensors (torch is only used for device memory and streams).

There is no fallback: if ``libanelm.so`` is missing or fails to load, every
entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libanelm.so")

ANELM_OK = 0
ANELM_F32 = 0
ANELM_F16 = 1
ROPE_INTERLEAVED = 0
ROPE_HALF_SPLIT = 1
DN_L2NORM = 1
DN_ORDER_TRANSFORMERS = 2
DN_GATED_NORM = 4
KV_TOKEN_MAJOR = 0
KV_HEAD_MAJOR = 1

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_IP = ctypes.POINTER(ctypes.c_int)
_FP = ctypes.POINTER(ctypes.c_float)

# name -> argtypes (restype is int for all but the query functions)
SIGNATURES = {
    "anelm_version": [],
    "anelm_device_cus": [],
    "anelm_stream_release": [_P],
    "anelm_rmsnorm": [_P, _P, _P, _I, _I, _I, _I, _F, _P],
    "anelm_rmsnorm_gated": [_P, _P, _P, _P, _I, _I, _P],
    "anelm_l2_normalize": [_P, _I, _I, _P],
    "anelm_apply_rope": [_P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _FP, _FP, _I, _P],
    "anelm_silu_inplace": [_P, _I, _P],
    "anelm_mul_sigmoid_inplace": [_P, _P, _I, _P],
    "anelm_softmax": [_P, _I, _I, _P],
    "anelm_matvec": [_P, _P, _P, _I, _I, _P],
    "anelm_conv1d_update": [_P, _P, _IP, _P, _P, _I, _I, _P],
    "anelm_gqa_attention": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P],
    "anelm_full_attn_decode": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F,
                               _I, _I, _FP, _FP, _IP, _IP, _I, _P],
    "anelm_full_attn_decode_kv": [_P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _I, _I, _I, _I, _I, _F, _F,
                                  _I, _I, _FP, _FP, _IP, _IP, _I, _P],
    "anelm_full_attn_decode_noalloc": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F,
                                       _I, _I, _FP, _FP, _IP, _IP, _I, _P],
    "anelm_attn_decode_paged": [_P, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P],
    "anelm_attn_decode_paged_step": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                                     _I, _I, _I, _I, _I, _F, _F, _I, _I, _P],
    "anelm_rope_table": [_P, _I, _I, _F],
    "anelm_attn_prefill": [_P, _I, _P, _P, _P, _I, _I, _I, _I, _P],
    "anelm_full_attn_prefill": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _F, _I, _I,
                                _P, _I, _IP, _IP, _I, _P],
    "anelm_deltanet_prefill_from_proj": [_P, _P, _P, _IP, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I,
                                         _P],
    "anelm_ssm_step": [_P, _P, _P, _P, _P, _F, _F, _I, _I, _I, _P],
    "anelm_deltanet_decode": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    "anelm_deltanet_decode_batched": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    "anelm_deltanet_decode_from_proj": [_P, _P, _P, _IP, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    "anelm_deltanet_prefill": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P],
    "anelm_lut6_unpack": [_P, _P, _I64, _P],
    "anelm_lut6_gemv": [_P, _P, _P, _P, _I, _I, _P],
    "anelm_lut6_proj": [_P, _P, _P, _P, _P, _F, _I, _I, _I, _P],
    "anelm_lut6_ffn": [_P, _P, _P, _F, _P, _P, _P, _P, _P, _P, _I, _I, _P],
    "anelm_lut6_gate_up": [_P, _P, _P, _P, _F, _P, _P, _P, _P, _I, _I, _P],
    "anelm_lut6_swiglu": [_P, _P, _P, _F, _P, _P, _P, _P, _I, _I, _P],
    "anelm_lut6_gemm": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "anelm_swiglu": [_P, _P, _P, _I64, _P],
    "anelm_swiglu_rows": [_P, _P, _I, _I, _P],
    "anelm_lut6_topk": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "anelm_sample_token": [_P, _P, _I, _P, _I, _F, _F, _I, _F, _F, _P],
    "anelm_hybrid_step_create": [ctypes.POINTER(_P), _P, _P, _I, _P, _P, _I, _P],
    "anelm_hybrid_step_run": [_P, _P],
    "anelm_hybrid_step_status": [_P, _IP],
    "anelm_hybrid_step_destroy": [_P],
    "anelm_hybrid_step_trace": [_P, _P, ctypes.c_size_t, _IP, _IP],
    "anelm_batch_step_create": [ctypes.POINTER(_P), _P, _P, _I, _P, _P],
    "anelm_batch_step_run": [_P, _I, _P],
    "anelm_batch_step_status": [_P, _IP],
    "anelm_batch_step_destroy": [_P],
    # compat tier (host pointers, synchronous)
    "anelm_cpu_silu_vec_inplace": [_P, _I, _P],
    "anelm_cpu_mul_sigmoid_inplace": [_P, _P, _I, _P],
    "anelm_cpu_rmsnorm": [_P, _P, _P, _I, _F],
    "anelm_cpu_rmsnorm_gated": [_P, _P, _P, _P, _I],
    "anelm_cpu_apply_rope_cached": [_P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P],
    "anelm_cpu_softmax": [_P, _I],
    "anelm_cpu_matvec": [_P, _P, _P, _I, _I],
    "anelm_cpu_l2_normalize": [_P, _I],
    "anelm_cpu_conv1d_update": [_P, _P, _IP, _P, _P, _I, _I],
    "anelm_cpu_ssm_step": [_P, _P, _P, _P, _P, _F, _F, _I, _I],
    "anelm_cpu_gqa_attention": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I],
}


class AnelmError(RuntimeError):
    """A libanelm call returned a non-zero status."""

    def __init__(self, fn: str, rc: int, msg: str):
        super().__init__(f"{fn} failed with status {rc}: {msg}")
        self.rc = rc


_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Loads libanelm.so (raises OSError if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise OSError(f"libanelm.so not built at {LIB_PATH}; run __graft_entry__.build()")
            L = ctypes.CDLL(LIB_PATH)
            L.anelm_last_error.restype = ctypes.c_char_p
            L.anelm_last_error.argtypes = []
            for name, args in SIGNATURES.items():
                f = getattr(L, name)
                f.argtypes = args
                f.restype = ctypes.c_int
            _lib = L
    return _lib


def last_error() -> str:
    return lib().anelm_last_error().decode()


def call(name: str, *args) -> None:
    """Calls a libanelm entry point and raises AnelmError on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != ANELM_OK:
        raise AnelmError(name, rc, last_error())


def status(name: str, *args) -> int:
    """Calls a libanelm entry point and returns its status code."""
    return getattr(lib(), name)(*args)


class HybridLayer(ctypes.Structure):
    """anelm_hybrid_layer (include/anelm.h)."""
    _fields_ = [("kind", _I),
                ("q_gate", _P), ("k", _P), ("v", _P), ("k_cache", _P), ("v_cache", _P),
                ("q_norm_w", _P), ("k_norm_w", _P),
                ("cache_start", _I), ("cache_len", _I), ("cache_capacity", _I), ("pos", _I),
                ("state", _P), ("dn_q", _P), ("dn_k", _P), ("dn_v", _P), ("dn_a", _P),
                ("dn_b", _P), ("dn_A", _P), ("dn_dt_bias", _P), ("dn_z", _P), ("dn_norm_w", _P),
                ("dn_flags", _I), ("core_out", _P),
                ("ffn_norm_w", _P), ("gate_w", _P), ("gate_lut", _P), ("up_w", _P),
                ("up_lut", _P), ("down_w", _P), ("down_lut", _P),
                ("in_norm_w", _P), ("first_w", _P), ("first_lut", _P), ("o_w", _P), ("o_lut", _P),
                ("proj", _P), ("conv_state", _P), ("conv_w", _P), ("conv_pos", _I)]


class HybridDims(ctypes.Structure):
    """anelm_hybrid_dims (include/anelm.h)."""
    _fields_ = [("hidden", _I), ("inter", _I), ("n_heads", _I), ("n_kv_heads", _I),
                ("head_dim", _I), ("rot_dim", _I), ("rope_mode", _I), ("theta", _F), ("eps", _F),
                ("lin_k_heads", _I), ("lin_v_heads", _I), ("lin_dim", _I), ("conv_kernel", _I)]


class BatchLayer(ctypes.Structure):
    """anelm_batch_layer (include/anelm.h)."""
    _fields_ = [("kind", _I),
                ("q_gate", _P), ("k", _P), ("v", _P), ("k_pages", _P), ("v_pages", _P), ("page_table", _P),
                ("q_norm_w", _P), ("k_norm_w", _P),
                ("state", _P), ("dn_q", _P), ("dn_k", _P), ("dn_v", _P), ("dn_a", _P), ("dn_b", _P),
                ("dn_A", _P), ("dn_dt_bias", _P), ("dn_z", _P), ("dn_norm_w", _P), ("dn_flags", _I),
                ("core_out", _P),
                ("ffn_norm_w", _P), ("gate_up_w", _P), ("gate_up_lut", _P), ("down_w", _P), ("down_lut", _P)]


class BatchSeqs(ctypes.Structure):
    """anelm_batch_seqs (include/anelm.h)."""
    _fields_ = [("n_seqs", _I), ("seq_lens", _P), ("positions", _P),
                ("page_size", _I), ("n_pages", _I), ("max_pages", _I), ("max_seq_len", _I),
                ("rope_table", _P), ("rope_rows", _I),
                ("final_norm_w", _P), ("lm_w", _P), ("lm_lut", _P), ("vocab", _I), ("top_k", _I),
                ("top_idx", _P), ("top_val", _P)]


LAYER_DELTANET = 0
LAYER_ATTENTION = 1
STEP_EAGER = 0
STEP_GRAPH = 1
STEP_PERSISTENT = 2
STEP_STATIC = 4
STEP_COOPERATIVE = 8

from . import ops  # noqa: E402,F401
