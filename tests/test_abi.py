"""CPU checks of the C ABI: libanelm.so loads, exports every entry point the
headers declare, and rejects bad arguments with a status code before any
device work (no compute calls here)."""
import ctypes
import os
import re
import subprocess

import pytest

from workloads import ROOT

HEADERS = [os.path.join(ROOT, "include", h) for h in ("anelm.h", "anelm_cpu_ops.h")]


def declared_symbols():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(anelm_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_headers_declare_entry_points():
    names = declared_symbols()
    assert "anelm_full_attn_decode" in names and "anelm_cpu_gqa_attention" in names
    assert len(names) >= 30


def test_library_exports_every_declared_symbol(anelm):
    lib_path = anelm.LIB_PATH
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\sT\s(anelm_\w+)", out))
    missing = [n for n in declared_symbols() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    # and the Python binding covers the same set
    bound = set(anelm.SIGNATURES) | {"anelm_last_error"}
    assert set(declared_symbols()) == bound


def test_cpp_compat_header_compiles_against_library(tmp_path, anelm):
    """A C++ caller written against core/cpu_ops.h's names builds and links
    with the drop-in header (compile + link only, nothing runs)."""
    src = tmp_path / "caller.cpp"
    src.write_text(
        '#include "anelm_cpu_ops.h"\n'
        "using namespace ane_lm;\n"
        "void step(float* out, float* q, const float* kc, const float* vc, float* y, float* st,\n"
        "          const float* k, const float* v, float* x, const float* w) {\n"
        "  rmsnorm(x, x, w, 256);\n"
        "  apply_rope_cached(q, x, 8, 2, 256, 512, 256, 64, 7, 1e7f, nullptr, nullptr);\n"
        "  gqa_attention(out, q, kc, vc, 8, 2, 256, 512, 0, 513, 2048);\n"
        "  ssm_step(y, st, q, k, v, 0.9f, sigmoid_f(0.3f), 128, 128);\n"
        "  l2_normalize(x, 128); softmax(x, 10); matvec(y, w, x, 4, 8);\n"
        "}\n")
    lib_dir = os.path.dirname(anelm.LIB_PATH)
    r = subprocess.run(["g++", "-std=c++17", "-shared", "-fPIC", "-I", os.path.join(ROOT, "include"),
                        str(src), "-L", lib_dir, "-lanelm", "-o", str(tmp_path / "libcaller.so")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_argument_validation_without_device(anelm):
    """Errors caught before any HIP call: NULL pointers and bad shapes."""
    st = anelm.status
    P = ctypes.c_void_p(16)   # a non-NULL dummy; never dereferenced on these paths
    assert st("anelm_rmsnorm", None, P, P, 8, 1, 8, 8, 1e-6, None) == -2
    assert st("anelm_rmsnorm", P, P, P, 0, 1, 8, 8, 1e-6, None) == -1
    assert "dim" in anelm.last_error()
    assert st("anelm_lut6_gemv", P, P, P, P, 33, 64, None) == -1        # out_dim % 32
    assert st("anelm_lut6_gemv", P, P, P, P, 64, 24, None) == -1        # in_dim % 16
    assert st("anelm_lut6_gemv", P, P, P, P, 64, 1 << 20, None) == -1   # in_dim too large
    assert st("anelm_lut6_topk", P, P, P, P, P, 1, 64, 64, 65, None) == -1  # k > 64
    assert st("anelm_gqa_attention", P, P, P, P, 1, 12, 4, 256, 512, 0, 10, 16, None) != 0  # G=3
    assert st("anelm_gqa_attention", P, P, P, P, 1, 8, 2, 96, 96, 0, 10, 16, None) == -1    # D=96
    assert st("anelm_gqa_attention", P, P, P, P, 1, 8, 2, 256, 512, 0, 17, 16, None) == -1  # len > cap
    assert st("anelm_gqa_attention", P, P, P, P, 7, 8, 2, 256, 512, 0, 10, 16, None) == -1  # dtype
    ring_s, ring_l = ctypes.c_int(0), ctypes.c_int(5)
    assert st("anelm_full_attn_decode", P, P, P, P, P, P, P, P, 8, 2, 256, 66 * 2 + 1, 0, 1e7,
              1e-6, 0, 1, None, None, ctypes.byref(ring_s), ctypes.byref(ring_l), 16, None) == -1
    assert (ring_s.value, ring_l.value) == (0, 5)   # ring untouched on error
    assert st("anelm_deltanet_decode", P, P, P, P, P, P, P, P, P, None, None, 16, 32, 64, 128, 1,
              None) == -1   # dk != 128
    assert st("anelm_deltanet_decode", P, P, P, P, P, P, P, P, P, None, None, 16, 24, 128, 128, 1,
              None) == -1   # Hv % Hk
    assert st("anelm_deltanet_decode", P, P, P, P, P, P, P, P, P, None, None, 16, 32, 128, 128, 8,
              None) == -1   # unknown flag
    assert st("anelm_deltanet_prefill", P, P, P, P, P, P, P, P, P, 16, 16, 32, 128, 128, 64, 4,
              None) == -1   # GATED_NORM is decode-only
    assert st("anelm_attn_prefill", P, 0, P, P, P, 64, 16, 4, 96, None) == -1
    assert st("anelm_lut6_unpack", P, P, 6, None) == -1
    assert st("anelm_attn_decode_paged", P, P, 256, P, P, P, P, 2, 4, 16, 8, 65, 16, 4, 256,
              None) == -1   # max_seq_len > max_pages * page_size
    assert st("anelm_apply_rope", P, P, 1, 1, 64, 64, 64, 66, 0, 1e7, None, None, 0, None) == -1
    assert st("anelm_cpu_rmsnorm", None, P, P, 4, 1e-6) == -2


def _persistent_layers(anelm, n=4):
    """Four layers (3 DeltaNet, 1 attention) whose every pointer is a
    non-NULL dummy (never dereferenced: creation fails before any device work)."""
    P = 16
    layers = (anelm.HybridLayer * n)()
    for i in range(n):
        L = layers[i]
        L.kind = anelm.LAYER_ATTENTION if (i + 1) % 4 == 0 else anelm.LAYER_DELTANET
        for name, typ in anelm.HybridLayer._fields_:
            if typ is ctypes.c_void_p and name not in ("in_norm_w", "first_w", "first_lut", "o_w", "o_lut",
                                                        "proj", "conv_state", "conv_w"):
                setattr(L, name, P)
        L.cache_capacity, L.cache_len, L.pos = 8192, 8191, 8191
        L.dn_flags = 5
    return layers


def test_persistent_step_rejects_before_device_work(anelm):
    """The persistent step refuses, at creation and before touching a device,
    a rotary width of 0 (the kernel reads a RoPE row unconditionally) and a
    layer without a pointer its kernel reads (e.g. no q/k norm weights)."""
    st = anelm.status
    dims = anelm.HybridDims(2560, 9216, 16, 4, 256, 64, 0, 1e7, 1e-6, 16, 32, 128, 4)
    h = ctypes.c_void_p()
    P = ctypes.c_void_p(16)
    for rot in (0, 3, 260):
        dims.rot_dim = rot
        layers = _persistent_layers(anelm)
        assert st("anelm_hybrid_step_create", ctypes.byref(h), ctypes.byref(dims), layers, 4, P, P,
                  anelm.STEP_PERSISTENT, None) == -1, rot
        assert "rot_dim" in anelm.last_error()
        assert not h.value
    dims.rot_dim = 64
    for name, layer in (("q_norm_w", 3), ("k_norm_w", 3), ("state", 0), ("down_lut", 1), ("dn_z", 2)):
        layers = _persistent_layers(anelm)
        setattr(layers[layer], name, None)
        assert st("anelm_hybrid_step_create", ctypes.byref(h), ctypes.byref(dims), layers, 4, P, P,
                  anelm.STEP_PERSISTENT, None) == -2, name
        assert f"layer {layer}" in anelm.last_error()
    # without the gated norm a DeltaNet layer needs no z / norm weight: the
    # pointer checks pass and only the device lookup can fail here
    layers = _persistent_layers(anelm)
    layers[2].dn_flags = 1
    layers[2].dn_z = None
    rc = st("anelm_hybrid_step_create", ctypes.byref(h), ctypes.byref(dims), layers, 4, P, P,
            anelm.STEP_PERSISTENT, None)
    assert rc not in (-1, -2), anelm.last_error()
    if rc == 0:   # a device was present: the step was built (nothing launched)
        anelm.call("anelm_hybrid_step_destroy", h)
