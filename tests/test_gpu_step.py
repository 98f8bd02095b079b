"""GPU parity of the hybrid decode step (models/llm/qwen3_5.cpp:1278-1356 over
the compute cores): the eager launch sequence against the oracle's layer loop,
and the one-launch persistent step against the eager step over several
advancing decode steps (ring append, ring wrap-around, DeltaNet state carry)."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import assert_close, to_dev, to_host
from workloads import QWEN35_08B, QWEN35_4B, hybrid_model, oracle_hybrid_step, widen

pytestmark = pytest.mark.gpu

_P = ctypes.c_void_p


def _p(t):
    return _P(t.data_ptr())


class DeviceModel:
    """Device copy of a HybridModel plus the anelm_hybrid_layer descriptors."""

    def __init__(self, anelm, m, dev):
        self.m = m
        d = m.dims
        self.keep = []
        self.outs = []
        self.layers = (anelm.HybridLayer * len(m.layers))()
        for i, L in enumerate(m.layers):
            t = {}
            for k, v in L.items():
                if isinstance(v, np.ndarray):
                    t[k] = to_dev(v, dev)
            out_len = d["n_heads"] * d["head_dim"] if L["kind"] == 1 else d["lin_v_heads"] * d["lin_dim"]
            t["core_out"] = torch.zeros(out_len, device=dev)
            D = self.layers[i]
            D.kind = L["kind"]
            for k, v in t.items():
                setattr(D, k, v.data_ptr())
            if L["kind"] == 1:
                D.cache_start, D.cache_len, D.cache_capacity, D.pos = L["start"], L["len"], L["cap"], L["pos"]
            else:
                D.dn_flags = L["dn_flags"]
            self.keep.append(t)
            self.outs.append(t["core_out"])
        self.x = to_dev(m.x, dev)
        self.h = torch.empty(2 * d["inter"], device=dev)

    def dims(self, anelm):
        d = self.m.dims
        return anelm.HybridDims(d["hidden"], d["inter"], d["n_heads"], d["n_kv_heads"], d["head_dim"],
                                d["rot_dim"], 0, d["theta"], d["eps"], d["lin_k_heads"], d["lin_v_heads"],
                                d["lin_dim"])


def _create(anelm, dm, mode, stream):
    h = _P()
    dims = dm.dims(anelm)
    rc = anelm.status("anelm_hybrid_step_create", ctypes.byref(h), ctypes.byref(dims), dm.layers,
                      len(dm.m.layers), _p(dm.x), _p(dm.h), mode, stream)
    return rc, h


def _stream():
    return _P(torch.cuda.current_stream().cuda_stream)


def test_eager_step_matches_oracle(anelm, orc, dev):
    """4 layers (3 DeltaNet, 1 attention) at the Qwen3.5-4B shape, one step."""
    m = hybrid_model(900, 4)
    dm = DeviceModel(anelm, m, dev)
    s = _stream()
    rc, h = _create(anelm, dm, anelm.STEP_EAGER, s)
    assert rc == 0, anelm.last_error()
    try:
        anelm.call("anelm_hybrid_step_run", h, s)
        outs = oracle_hybrid_step(orc, m)
        for i, L in enumerate(m.layers):
            assert_close(to_host(dm.outs[i]), outs[i], what=f"layer {i} core output")
            if L["kind"] == 0:
                assert_close(to_host(dm.keep[i]["state"]), L["state"], what=f"layer {i} state")
            else:
                slot = (L["start"] + L["len"] - 1) % L["cap"]
                for name in ("k_cache", "v_cache"):
                    got = widen(to_host(dm.keep[i][name])[slot])
                    assert_close(got, widen(L[name][slot]), what=f"layer {i} {name} appended row")
        assert_close(to_host(dm.x), m.x, what="hidden state after 4 layers")
    finally:
        anelm.call("anelm_hybrid_step_destroy", h)


def _check_against_oracle(anelm, orc, dm, h, m, s, steps, x_rel, x_abs, label, persistent):
    """Runs `steps` advancing steps of the created step `h` and, after each,
    one oracle step on the host model `m`: every layer's core output,
    DeltaNet state and appended K / V row at the parity bar, x at
    (x_rel, x_abs)."""
    for step in range(steps):
        print(f"{label}: step {step}", flush=True)
        anelm.call("anelm_hybrid_step_run", h, s)
        torch.cuda.synchronize()
        if persistent:
            st = ctypes.c_int(-1)
            anelm.call("anelm_hybrid_step_status", h, ctypes.byref(st))
            assert st.value == 0, "a grid barrier timed out"
        outs = oracle_hybrid_step(orc, m)
        for i, L in enumerate(m.layers):
            assert_close(to_host(dm.outs[i]), outs[i], what=f"{label} step {step} layer {i} core output")
            if L["kind"] == 0:
                assert_close(to_host(dm.keep[i]["state"]), L["state"], what=f"{label} step {step} layer {i} state")
            else:
                slot = (L["start"] + L["len"] - 1) % L["cap"]
                for name in ("k_cache", "v_cache"):
                    got = widen(to_host(dm.keep[i][name][slot]))
                    assert_close(got, widen(L[name][slot]), what=f"{label} step {step} layer {i} {name} row {slot}")
        assert_close(to_host(dm.x), m.x, rel=x_rel, max_abs=x_abs, what=f"{label} step {step} hidden state")


def _persistent_or_skip(anelm, dm, s):
    rc, h = _create(anelm, dm, anelm.STEP_PERSISTENT, s)
    if rc != 0:
        pytest.skip(f"persistent step unsupported here: {anelm.last_error()}")
    return h


# 32 layers at the benchmark's shape (Qwen3.5-4B, ctx 8192): one ring one key
# short of full (the step fills it), one full ring that wraps (the new key
# overwrites the oldest slot 100), the rest at 5000 keys.
_C4_RINGS = [(0, 8191), (100, 8192)] + [(0, 5000)] * 6


def test_persistent_step_matches_oracle_c4(anelm, orc, dev):
    """The timed one-launch step at the benchmark's configuration (32 layers,
    LUTs ~ N(0, 0.02)) against the oracle's layer loop.  The cores' inputs do
    not depend on x, so every layer's core output, DeltaNet state and
    appended K / V row is held to the parity bar at all 32 layers.  x itself
    is chaotic at this LUT scale: the fp16 roundings of the FFN inputs turn a
    1e-7 relative nudge of the oracle's own x into a 1.6e-3 rel-L2 change
    (0.039 max-abs, |x| up to 24) after 32 layers, so x is held to rel-L2
    2e-2 and max-abs 0.5 here; the test below checks x at the parity bar."""
    m = hybrid_model(902, 32, rings=_C4_RINGS)
    dm = DeviceModel(anelm, m, dev)
    s = _stream()
    h = _persistent_or_skip(anelm, dm, s)
    try:
        _check_against_oracle(anelm, orc, dm, h, m, s, 1, 2e-2, 0.5, "C4 32 layers", True)
    finally:
        anelm.call("anelm_hybrid_step_destroy", h)


def test_persistent_step_matches_oracle_32_layers_x(anelm, orc, dev):
    """32 layers with LUTs ~ N(0, 0.005): the same 1e-7 nudge moves the
    oracle's x by 1.9e-5 rel-L2 after 32 layers, so x -- the FFN chain through
    every layer -- is held to the parity bar (rel-L2 1e-3, max-abs 2e-2)."""
    m = hybrid_model(903, 32, rings=_C4_RINGS, lut_std=0.005)
    dm = DeviceModel(anelm, m, dev)
    s = _stream()
    h = _persistent_or_skip(anelm, dm, s)
    try:
        _check_against_oracle(anelm, orc, dm, h, m, s, 1, 1e-3, 2e-2, "32 layers lut 0.005", True)
    finally:
        anelm.call("anelm_hybrid_step_destroy", h)


def test_persistent_step_advancing_matches_oracle(anelm, orc, dev):
    """8 layers, 3 advancing steps against the oracle: ring append, the
    full ring wrapping (slot 8000 onwards), DeltaNet states carried."""
    m = hybrid_model(904, 8, rings=[(0, 5000), (8000, 8192)], lut_std=0.005)
    dm = DeviceModel(anelm, m, dev)
    s = _stream()
    h = _persistent_or_skip(anelm, dm, s)
    try:
        _check_against_oracle(anelm, orc, dm, h, m, s, 3, 1e-3, 2e-2, "8 layers advancing", True)
    finally:
        anelm.call("anelm_hybrid_step_destroy", h)


@pytest.mark.parametrize("flags", [1 | 4, 1 | 2 | 4, 0, 1, 2 | 4])
def test_persistent_step_deltanet_flags(anelm, orc, dev, flags):
    """Every DeltaNet branch of the one-launch step against the oracle:
    l2 norm on / off, cpu_ops or decay-first order, gated norm or plain
    output (4 layers: 3 DeltaNet + 1 attention)."""
    m = hybrid_model(905 + flags, 4, rings=[(0, 7000)], lut_std=0.005, dn_flags=flags)
    dm = DeviceModel(anelm, m, dev)
    s = _stream()
    h = _persistent_or_skip(anelm, dm, s)
    try:
        _check_against_oracle(anelm, orc, dm, h, m, s, 2, 1e-3, 2e-2, f"flags {flags}", True)
    finally:
        anelm.call("anelm_hybrid_step_destroy", h)


def test_graph_step_survives_workspace_growth(anelm, orc, dev):
    """The HIP-graph step after the library workspace has grown (a top-k
    over 512 x 262144 logits needs 512 MiB of it, freeing the old buffer):
    its attention layers use partial buffers the step owns, so one replay
    matches the oracle's step.  Creating the step runs nothing (x, states
    and rings are unchanged at create)."""
    m = hybrid_model(906, 4, rings=[(0, 3000)], lut_std=0.005)
    dm = DeviceModel(anelm, m, dev)
    x0 = to_host(dm.x).copy()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        _graph_after_growth(anelm, orc, dev, dm, m, x0)


def _graph_after_growth(anelm, orc, dev, dm, m, x0):
    s = _stream()   # the side stream (graph capture needs a non-null stream)
    rc, h = _create(anelm, dm, anelm.STEP_GRAPH, s)
    assert rc == 0, anelm.last_error()
    try:
        torch.cuda.synchronize()
        assert np.array_equal(to_host(dm.x), x0), "create ran a step"
        from workloads import lut6_matrix
        pk, lut, _ = lut6_matrix(907, 262144, 64)
        xb = torch.randn(512, 64, device=dev)
        anelm.ops.lut6_topk(to_dev(pk, dev), to_dev(lut, dev), xb, 262144, 64, 8)
        torch.cuda.synchronize()
        _check_against_oracle(anelm, orc, dm, h, m, s, 1, 1e-3, 2e-2, "graph after workspace growth", False)
    finally:
        anelm.call("anelm_hybrid_step_destroy", h)


def _persistent_vs_eager(anelm, m, dev, steps, label, extra_mode=0):
    """Runs `steps` advancing decode steps of model m through the eager path
    and the persistent step side by side and compares every core output,
    state, cache and the hidden state after each."""
    a = DeviceModel(anelm, m, dev)
    b = DeviceModel(anelm, m, dev)
    s = _stream()
    rc, ha = _create(anelm, a, anelm.STEP_EAGER, s)
    assert rc == 0, anelm.last_error()
    rc, hb = _create(anelm, b, anelm.STEP_PERSISTENT | extra_mode, s)
    if rc != 0:
        anelm.call("anelm_hybrid_step_destroy", ha)
        pytest.skip(f"persistent step unsupported here: {anelm.last_error()}")
    try:
        for step in range(steps):
            print(f"{label}: persistent step {step}", flush=True)
            anelm.call("anelm_hybrid_step_run", ha, s)
            anelm.call("anelm_hybrid_step_run", hb, s)
            torch.cuda.synchronize()
            st = ctypes.c_int(-1)
            anelm.call("anelm_hybrid_step_status", hb, ctypes.byref(st))
            assert st.value == 0, "a grid barrier timed out"
            for i, L in enumerate(m.layers):
                assert_close(to_host(b.outs[i]), to_host(a.outs[i]), what=f"step {step} layer {i} core")
                if L["kind"] == 0:
                    assert_close(to_host(b.keep[i]["state"]), to_host(a.keep[i]["state"]),
                                 what=f"step {step} layer {i} state")
                else:
                    for name in ("k_cache", "v_cache"):
                        assert_close(widen(to_host(b.keep[i][name])), widen(to_host(a.keep[i][name])),
                                     what=f"step {step} layer {i} {name}")
            assert_close(to_host(b.x), to_host(a.x), rel=1e-4, max_abs=1e-3, what=f"step {step} hidden state")
    finally:
        anelm.call("anelm_hybrid_step_destroy", ha)
        anelm.call("anelm_hybrid_step_destroy", hb)


def test_persistent_step_matches_eager(anelm, dev):
    """8 layers, 3 advancing decode steps: one ring mid-fill (5000 of 8192
    keys), one full ring that wraps and overwrites its oldest slot.

    LUTs ~ N(0, 0.005): with the 0.02 scale of the other tests, eight random
    FFN blocks amplify any fp32 summation-order difference through the fp16
    activation roundings (a 1e-7 relative nudge of x moves the oracle's own x
    by 7e-4 after one step); at 0.005 the same nudge moves it by < 2e-5 over
    three steps while the FFNs still change x by 4% per step, so the hidden
    state is checked at 1e-4."""
    m = hybrid_model(901, 8, rings=[(0, 5000), (8000, 8192)], lut_std=0.005)
    _persistent_vs_eager(anelm, m, dev, 3, "8 layers")


def test_persistent_step_cooperative_launch(anelm, dev):
    """The cooperative launch (the runtime admits the grid only when every
    workgroup can be resident) runs the same kernel: 3 advancing steps
    against the eager path."""
    m = hybrid_model(908, 4, rings=[(0, 5000)], lut_std=0.005)
    _persistent_vs_eager(anelm, m, dev, 3, "cooperative", anelm.STEP_COOPERATIVE)


def test_persistent_step_rope_table_growth(anelm, dev):
    """The persistent step advances its own descriptors on the device and
    reads RoPE rows from a table sized in 4096-position blocks; starting at
    position 4094, the second step needs row 4096, so the table grows (the
    host waits for the launch before, rebuilds and re-uploads) between steps."""
    m = hybrid_model(905, 4, rings=[(0, 4094)], lut_std=0.005)
    _persistent_vs_eager(anelm, m, dev, 3, "table growth")


def test_persistent_step_08b_shape_matches_oracle(anelm, orc, dev):
    """The reference's default model shape (Qwen3.5-0.8B, qwen3_5.h:51-69:
    hidden 1024, inter 3584, 8 q / 2 kv heads, 16 value heads) as one
    persistent launch on the 256-CU grid: attention uses 128 of the
    workgroups and the DeltaNet cores 128, the rest only join the barriers.
    8 layers, one step against the oracle."""
    m = hybrid_model(906, 8, dims=QWEN35_08B, rings=[(0, 3000), (8000, 8192)])
    dm = DeviceModel(anelm, m, dev)
    s = _stream()
    h = _persistent_or_skip(anelm, dm, s)
    try:
        _check_against_oracle(anelm, orc, dm, h, m, s, 1, 1e-3, 2e-2, "0.8B shape", True)
    finally:
        anelm.call("anelm_hybrid_step_destroy", h)


def test_persistent_step_08b_shape_advancing_matches_eager(anelm, dev):
    """The 0.8B shape, 3 advancing steps (one ring mid-fill, one wrapping)
    against the eager path."""
    m = hybrid_model(907, 8, dims=QWEN35_08B, rings=[(0, 3000), (8000, 8192)], lut_std=0.005)
    _persistent_vs_eager(anelm, m, dev, 3, "0.8B shape")

