"""Concurrent calls on two streams: the library's scratch (split partials,
merge records, arrival counters, chunk records) belongs to one (device,
stream) pair, so decode attention, causal prefill attention and the chunked
DeltaNet prefill issued on two streams at once give the bit-identical
results of the same calls issued one after another -- the reference's
cpu_ops functions keep no mutable globals (core/cpu_ops.cpp:1-206) -- and
those match the oracle."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import assert_close, to_dev, to_host
from workloads import attn_decode_case, deltanet_case, prefill_inputs

pytestmark = pytest.mark.gpu


class Work:
    """One set of inputs for the three calls; run() issues them on the
    current stream from fresh copies of the mutable buffers."""

    def __init__(self, seed, dev):
        # 901 keys over a wrapped ring: 15 key splits of 64, merged in the
        # kernel through the stream's arrival counters
        self.c = attn_decode_case(seed, n_heads=16, n_kv_heads=4, head_dim=256, cached=900,
                                  capacity=2048, start=1500)
        c = self.c
        self.dq, self.dk, self.dv = (to_dev(c.q_gate, dev), to_dev(c.k, dev), to_dev(c.v, dev))
        self.kc, self.vc = to_dev(c.k_cache, dev), to_dev(c.v_cache, dev)
        self.qw, self.kw = to_dev(c.q_norm_w, dev), to_dev(c.k_norm_w, dev)
        self.pq, self.pk, self.pv = (to_dev(a, dev) for a in prefill_inputs(seed + 1, 700, 16, 4, 256))
        self.pin = prefill_inputs(seed + 1, 700, 16, 4, 256)
        self.dn = deltanet_case(seed + 2, Hk=16, Hv=32, S=256)
        self.dd = {k: to_dev(getattr(self.dn, k), dev) for k in ("state", "q", "k", "v", "a", "b", "A",
                                                                 "dt_bias")}

    def parts(self, anelm):
        """The three calls as closures (each issues on the current stream)."""
        c, d = self.c, self.dd
        res = {}

        def decode():
            kc, vc = self.kc.clone(), self.vc.clone()
            ring = anelm.ops.KVRing(c.capacity, c.start, c.length)
            res["dec"] = anelm.ops.full_attn_decode(self.dq, self.dk, self.dv, kc, vc, self.qw, self.kw, ring,
                                                    c.n_heads, c.n_kv_heads, c.head_dim, c.rot_dim, c.pos,
                                                    c.theta, c.eps)

        def prefill():
            res["pre"] = anelm.ops.attn_prefill(self.pq, self.pk, self.pv)

        def deltanet():
            res["st"] = d["state"].clone()
            res["y"] = anelm.ops.deltanet_prefill(res["st"], d["q"], d["k"], d["v"], d["a"], d["b"], d["A"],
                                                  d["dt_bias"], 1)

        return res, [decode, prefill, deltanet]

    def run(self, anelm):
        res, calls = self.parts(anelm)
        for f in calls:
            f()
        return res["dec"], res["pre"], res["y"], res["st"]


def _host(outs):
    return [to_host(t) for t in outs]


def test_two_streams_match_serial_calls(anelm, orc, dev):
    works = [Work(1500, dev), Work(1600, dev)]
    serial = [_host(w.run(anelm)) for w in works]
    # against the oracle (the serial results; the concurrent ones are compared
    # bit for bit with these below)
    for w, (dec, pre, y, st) in zip(works, serial):
        c = w.c
        want = orc.full_attn_decode(c.q_gate, c.k, c.v, c.k_cache, c.v_cache, c.q_norm_w, c.k_norm_w,
                                    c.n_heads, c.n_kv_heads, c.head_dim, c.rot_dim, c.pos, c.theta, c.eps,
                                    0, True, c.start, c.length, c.capacity)[0]
        assert_close(dec, want, what="decode attention")
        q, k, v = w.pin
        for t in (0, 350, 699):
            assert_close(pre[t], orc.prefill_attention(q, k, v, t, t + 1)[0], what=f"prefill row {t}")
        n = w.dn
        yw, sw = orc.deltanet_prefill(n.state[:2], n.q[:, :1], n.k[:, :1], n.v[:, :2], n.a[:, :2], n.b[:, :2],
                                      n.A[:2], n.dt_bias[:2], 1)
        assert_close(y[:, :2], yw, what="deltanet prefill y (value heads 0, 1)")
        assert_close(st[:2], sw, what="deltanet prefill state (value heads 0, 1)")
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    try:
        for rep in range(3):
            print(f"two streams, round {rep}", flush=True)
            torch.cuda.synchronize()
            # the two streams' calls are issued alternately without waits, so
            # their kernels overlap on the device
            parts = [w.parts(anelm) for w in works]
            for k in range(3):
                for i in (0, 1):
                    with torch.cuda.stream(streams[i]):
                        parts[i][1][k]()
            torch.cuda.synchronize()
            outs = [(r["dec"], r["pre"], r["y"], r["st"]) for r, _ in parts]
            for i in (0, 1):
                for name, got, want in zip(("decode", "prefill", "deltanet y", "deltanet state"),
                                           _host(outs[i]), serial[i]):
                    assert np.array_equal(got, want), f"round {rep} stream {i}: {name} differs from the serial call"
    finally:
        for s in streams:
            anelm.call("anelm_stream_release", ctypes.c_void_p(s.cuda_stream))
