"""anelm_full_attn_decode_noalloc (the allocation-free variant of
anelm_full_attn_decode, split partials in a static per-device array) against
anelm_full_attn_decode through the C ABI: two calls in a row, the second with
a smaller input, bit-identical outputs, cache rows and ring state; device
memory unchanged across the calls; oversize calls rejected with ANELM_ERANGE."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import to_dev, to_host
from workloads import attn_decode_case

pytestmark = pytest.mark.gpu

_P = ctypes.c_void_p
ANELM_ERANGE = -4


def _call(anelm, name, c, dev, out, kc, vc, ring):
    """One decode step of case c through entry point `name` (ring: [start, len])."""
    start, length = ctypes.c_int(ring[0]), ctypes.c_int(ring[1])
    keep = [to_dev(a, dev) for a in (c.q_gate, c.k, c.v, c.q_norm_w, c.k_norm_w)]
    qg, k, v, qn, kn = keep
    rc = anelm.status(name, _P(out.data_ptr()), _P(qg.data_ptr()), _P(k.data_ptr()), _P(v.data_ptr()),
                      _P(kc.data_ptr()), _P(vc.data_ptr()), _P(qn.data_ptr()), _P(kn.data_ptr()),
                      c.n_heads, c.n_kv_heads, c.head_dim, c.rot_dim, c.pos, ctypes.c_float(c.theta),
                      ctypes.c_float(c.eps), 0, 1, None, None, ctypes.byref(start), ctypes.byref(length),
                      c.capacity, _P(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return rc, (start.value, length.value)


def _compare(anelm, c, dev, label):
    outs, caches, rings = [], [], []
    for name in ("anelm_full_attn_decode", "anelm_full_attn_decode_noalloc"):
        out = torch.full((c.n_heads, c.head_dim), float("nan"), device=dev)
        kc, vc = to_dev(c.k_cache, dev), to_dev(c.v_cache, dev)
        rc, ring = _call(anelm, name, c, dev, out, kc, vc, (c.start, c.length))
        assert rc == 0, f"{label} {name}: {anelm.last_error()}"
        outs.append(to_host(out))
        caches.append((to_host(kc), to_host(vc)))
        rings.append(ring)
    assert np.array_equal(outs[1], outs[0]), f"{label}: outputs differ"
    assert np.array_equal(caches[1][0], caches[0][0]) and np.array_equal(caches[1][1], caches[0][1]), \
        f"{label}: caches differ"
    assert rings[1] == rings[0], f"{label}: ring state differs"


def test_noalloc_matches_full_attn_decode(anelm, dev):
    # 4B shape over a full 8192-key ring that wraps (128 splits per kv head)
    big = attn_decode_case(950, n_heads=16, n_kv_heads=4, cached=8192, capacity=8192, start=37)
    print("noalloc: 16q/4kv D256, 8192-key wrapping ring", flush=True)
    _compare(anelm, big, dev, "16q/4kv 8192 keys")
    free0, _ = torch.cuda.mem_get_info()
    # then a smaller call: 0.8B shape, 513 keys (9 splits), stale partials of
    # the first call still in the array
    small = attn_decode_case(951)
    print("noalloc: 8q/2kv D256, 513 keys", flush=True)
    _compare(anelm, small, dev, "8q/2kv 513 keys")
    one = attn_decode_case(952, cached=40)   # one split: no partials at all
    print("noalloc: 8q/2kv D256, 41 keys", flush=True)
    _compare(anelm, one, dev, "8q/2kv 41 keys")
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, f"device memory changed by {free0 - free1} bytes across the calls"


def test_noalloc_rejects_oversize(anelm, dev):
    """40000 keys at 16 q / 4 kv heads need 10.3 MB of partials > 8 MiB."""
    c = attn_decode_case(953, n_heads=16, n_kv_heads=4, cached=8, capacity=40000)
    c.length = 39999
    out = torch.empty(c.n_heads, c.head_dim, device=dev)
    kc = torch.zeros(8, device=dev)   # never touched: the size check comes first
    rc, ring = _call(anelm, "anelm_full_attn_decode_noalloc", c, dev, out, kc, kc, (0, 39999))
    assert rc == ANELM_ERANGE, (rc, anelm.last_error())
    assert ring == (0, 39999)
