"""A stream_generate-shaped decode loop (generate.cpp:30-218; the model
forward of models/llm/qwen3_5.cpp:1278-1417) driven through the C ABI: per
token the embedding row, ONE anelm_hybrid_step run over complete layers
(input norm + first projection, the conv ring + DeltaNet core or the
attention core, o_proj + residual, FFN), the final norm, the LUT6 LM head and
anelm_sample_token with the reference's default penalties
(core/sampling.h:7-12) -- compared token by token with the oracle's decode
loop on the same random-init model."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import assert_close, to_dev, to_host
from workloads import QWEN35_4B, TINY_LM, OracleLM, tiny_lm

pytestmark = pytest.mark.gpu

_P = ctypes.c_void_p


class StepLM:
    """The tiny LM's layers as anelm_hybrid_layer descriptors with projections."""

    def __init__(self, anelm, m, dev, mode=0):
        self.anelm, self.m, self.dev = anelm, m, dev
        d = m["dims"]
        H, I = d["hidden"], d["inter"]
        Hq, Hkv, D = d["n_heads"], d["n_kv_heads"], d["head_dim"]
        Hk, Hv, dl = d["lin_k_heads"], d["lin_v_heads"], d["lin_dim"]
        qkv = 2 * Hk * dl + Hv * dl
        self.keep = []
        n = len(m["layers"])
        self.layers = (anelm.HybridLayer * n)()

        def put(t):
            self.keep.append(t)
            return t.data_ptr()

        def dv(a):
            return put(to_dev(a, dev))

        for i, L in enumerate(m["layers"]):
            S = self.layers[i]
            S.kind = 1 if L["attn"] else 0
            S.in_norm_w = dv(L["in_norm"])
            S.first_w, S.first_lut = dv(L["first"][0]), dv(L["first"][1])
            S.o_w, S.o_lut = dv(L["o"][0]), dv(L["o"][1])
            S.proj = put(torch.zeros(L["first"][1].shape[0] * 32, device=dev))
            S.ffn_norm_w = dv(L["post_norm"])
            S.gate_w, S.gate_lut = dv(L["gate"][0]), dv(L["gate"][1])
            S.up_w, S.up_lut = dv(L["up"][0]), dv(L["up"][1])
            S.down_w, S.down_lut = dv(L["down"][0]), dv(L["down"][1])
            if L["attn"]:
                shape = (d["cap"], Hkv, D)
                S.k_cache = put(torch.zeros(shape, dtype=torch.float16, device=dev))
                S.v_cache = put(torch.zeros(shape, dtype=torch.float16, device=dev))
                S.q_norm_w, S.k_norm_w = dv(L["q_norm"]), dv(L["k_norm"])
                S.cache_start, S.cache_len, S.cache_capacity, S.pos = 0, 0, d["cap"], 0
                S.core_out = put(torch.zeros(Hq * D, device=dev))
            else:
                S.state = put(torch.zeros(Hv, dl, dl, device=dev))
                S.conv_state = put(torch.zeros(qkv, d["conv_kernel"] - 1, device=dev))
                S.conv_w = dv(L["conv_w"])
                S.dn_A, S.dn_dt_bias, S.dn_norm_w = dv(L["A"]), dv(L["dt_bias"]), dv(L["norm_w"])
                S.dn_flags = 1 | 4
                S.conv_pos = 0
                S.core_out = put(torch.zeros(Hv * dl, device=dev))
        self.x = torch.zeros(H, device=dev)
        self.h = torch.zeros(2 * I, device=dev)
        self.dims = anelm.HybridDims(H, I, Hq, Hkv, D, d["rot_dim"], 0, d["theta"], d["eps"], Hk, Hv, dl,
                                     d["conv_kernel"])
        self.embed = to_dev(m["embed"], dev)
        self.final_norm = to_dev(m["final_norm"], dev)
        self.lm = tuple(to_dev(a, dev) for a in m["lm_head"])
        self.stream = _P(torch.cuda.current_stream().cuda_stream)
        self.handle = _P()
        anelm.call("anelm_hybrid_step_create", ctypes.byref(self.handle), ctypes.byref(self.dims), self.layers,
                   n, _P(self.x.data_ptr()), _P(self.h.data_ptr()), mode, self.stream)

    def close(self):
        self.anelm.call("anelm_hybrid_step_destroy", self.handle)

    def forward(self, token):
        """Qwen35Model::forward: embedding row, the layer loop, final norm, LM head."""
        d = self.m["dims"]
        self.x.copy_(self.embed[token])
        self.anelm.call("anelm_hybrid_step_run", self.handle, self.stream)
        xf = self.anelm.ops.rmsnorm(self.x, self.final_norm, d["eps"])
        lw, ll = self.lm
        return self.anelm.ops.lut6_gemv(lw, ll, xf, d["vocab"], d["hidden"])


def _generate(anelm, orc, m, dev, steps, T, draws):
    """Both loops side by side; each emitted token feeds the next step and
    joins the penalty window (generate.cpp:30-218 with sample_token)."""
    ref, gpu = OracleLM(orc, m), StepLM(anelm, m, dev)
    recent, forced = [], 0
    tok = 1
    try:
        for pos in range(steps):
            tok_ref_in = tok
            _, logits_ref = ref.step(tok_ref_in, pos)
            logits_gpu = gpu.forward(tok_ref_in)
            assert_close(to_host(logits_gpu), logits_ref, what=f"logits at step {pos}")
            r = float(draws[pos])
            want, adj = orc.sample_token(logits_ref, np.array(recent, np.int32), T, 1.2, 256, 0.1, r)
            rec = to_dev(np.array(recent, np.int32), dev) if recent else None
            got = int(to_host(anelm.ops.sample_token(logits_gpu, rec, T, 1.2, 256, 0.1, r))[0])
            if T > 0:
                # the device draws on the exact running sum of the softmax, the
                # reference on a sequential fp32 one (their crossings can differ
                # by rounding; see test_gpu_sampling.py)
                rf = float(np.float32(r))
                _, pen = orc.sample_token(to_host(logits_gpu), np.array(recent, np.int32), 0.0, 1.2, 256, 0.1,
                                          0.5)
                z = (pen * (np.float32(1.0) / np.float32(T))).astype(np.float64)
                p = np.exp(z - z.max())
                cum = np.cumsum(p / p.sum())
                lo = cum[got - 1] if got > 0 else 0.0
                assert max(0.0, lo - rf, rf - cum[got]) <= 2e-6, f"step {pos}: GPU token {got} off the exact CDF"
                undecided = got != want      # the logits' rounding or the oracle's fp32 sums chose a neighbour
            else:
                top2 = np.sort(adj)[-2:]
                undecided = top2[1] - top2[0] < 1e-3
                if not undecided:
                    assert got == want, f"step {pos}: GPU token {got} != oracle token {want}"
            forced += bool(undecided)        # the oracle's token feeds both loops
            tok = want
            recent.append(tok)
    finally:
        gpu.close()
    return recent, forced


def test_generate_greedy_with_penalties_64(anelm, orc, dev):
    m = tiny_lm(2025)
    toks, forced = _generate(anelm, orc, m, dev, 64, 0.0, np.zeros(64))
    assert forced <= 2 and len(set(toks)) > 4, (forced, toks)


def test_generate_greedy_exact_64(anelm, orc, dev):
    """The 64-token greedy gate through the product step: two independent
    loops (each feeds its OWN tokens back), greedy with the reference's
    default penalties, must emit identical tokens.  The seed is checked
    first: the oracle's smallest top-2 gap of the penalised logits over the
    64 decisions is ~8e-3, far above the ~1e-6 relative GPU/oracle logit
    difference, so every token is decided."""
    m = tiny_lm(2042)
    ref = OracleLM(orc, m)
    want, gaps, tok = [], [], 1
    for pos in range(64):
        _, logits = ref.step(tok, pos)
        tok, adj = orc.sample_token(logits, np.array(want, np.int32), 0.0, 1.2, 256, 0.1, 0.5)
        top2 = np.sort(adj)[-2:]
        gaps.append(float(top2[1] - top2[0]))
        want.append(tok)
    assert min(gaps) > 1e-3, "seeded model has a near-tie: pick another seed"
    gpu = StepLM(anelm, m, dev, mode=anelm.STEP_EAGER)
    got, tok = [], 1
    try:
        for pos in range(64):
            logits = gpu.forward(tok)
            rec = to_dev(np.array(got, np.int32), dev) if got else None
            tok = int(to_host(anelm.ops.sample_token(logits, rec, 0.0, 1.2, 256, 0.1, 0.5))[0])
            got.append(tok)
    finally:
        gpu.close()
    assert got == want, next(i for i, (a, b) in enumerate(zip(got, want)) if a != b)


def test_generate_sampled_t06(anelm, orc, dev):
    """Temperature 0.6 with seeded uniform draws (the reference's drand48)."""
    m = tiny_lm(2026)
    draws = np.random.default_rng(2027).uniform(0, 1, 48)
    toks, forced = _generate(anelm, orc, m, dev, 48, 0.6, draws)
    assert forced <= 4 and len(set(toks)) > 4, (forced, toks)


def test_complete_layers_4b_shape(anelm, orc, dev):
    """Four complete layers (3 DeltaNet + 1 attention) at the Qwen3.5-4B shape
    -- first projections 2560->12352 / 2560->10240, o_proj 4096->2560, FFN
    2560->9216->2560 -- three decode steps; the hidden state after the layer
    loop against the oracle's."""
    m = tiny_lm(2028, dims=_DIMS_4B)
    ref, gpu = OracleLM(orc, m), StepLM(anelm, m, dev)
    try:
        for pos, tok in enumerate((3, 17, 101)):
            _, logits_ref = ref.step(tok, pos)
            logits_gpu = gpu.forward(tok)
            assert_close(to_host(logits_gpu), logits_ref, what=f"4B-shape logits at step {pos}")
    finally:
        gpu.close()


_DIMS_4B = dict(TINY_LM, hidden=QWEN35_4B["hidden"], inter=QWEN35_4B["inter"], n_heads=16, n_kv_heads=4,
                lin_k_heads=16, lin_v_heads=32, vocab=256, cap=64)
_DIMS_08B = dict(TINY_LM, hidden=1024, inter=3584, n_heads=8, n_kv_heads=2, lin_k_heads=16, lin_v_heads=16)


def _persistent_lm(anelm, m, dev):
    gpu = StepLM.__new__(StepLM)
    try:
        StepLM.__init__(gpu, anelm, m, dev, mode=anelm.STEP_PERSISTENT)
    except Exception as e:   # noqa: BLE001 -- a device without 256 CUs
        pytest.skip(f"persistent step unsupported here: {e}")
    return gpu


_PROJ_OFF = pytest.mark.skip(reason="complete layers in one persistent launch are switched off: a run of a "
                             "variant of step_kernel_proj ended in a GPU fault whose cause is not found")


@_PROJ_OFF
def test_complete_layers_persistent_4b_shape(anelm, orc, dev):
    """The complete layers as ONE persistent launch per step (first
    projection, conv ring + DeltaNet core or attention core with its merge,
    o_proj + residual, FFN: five grid-barrier phases per layer) at the
    Qwen3.5-4B shape, four layers, three decode steps: the logits against
    the oracle's Qwen35Model::forward."""
    m = tiny_lm(2028, dims=_DIMS_4B)
    ref, gpu = OracleLM(orc, m), _persistent_lm(anelm, m, dev)
    try:
        for pos, tok in enumerate((3, 17, 101)):
            _, logits_ref = ref.step(tok, pos)
            logits_gpu = gpu.forward(tok)
            assert_close(to_host(logits_gpu), logits_ref, what=f"persistent 4B-shape logits at step {pos}")
        st = ctypes.c_int(-1)
        anelm.call("anelm_hybrid_step_status", gpu.handle, ctypes.byref(st))
        assert st.value == 0, "a grid barrier timed out"
    finally:
        gpu.close()


@_PROJ_OFF
def test_complete_layers_persistent_matches_eager(anelm, dev):
    """Eight complete layers at the 4B shape, five decode steps (the conv
    rings cycle past their 3 slots, the KV rings fill): the persistent step's
    hidden state, caches, conv rings and DeltaNet states against the eager
    executor's."""
    m = tiny_lm(2032, dims=dict(_DIMS_4B, layers=8), lut_std=0.005)
    a = StepLM(anelm, m, dev, mode=anelm.STEP_EAGER)
    b = _persistent_lm(anelm, m, dev)
    try:
        for pos, tok in enumerate((5, 9, 200, 31, 77)):
            xa = to_host(a.forward(tok))
            xb = to_host(b.forward(tok))
            torch.cuda.synchronize()
            assert_close(xb, xa, what=f"step {pos} logits")
            for i, (ta, tb) in enumerate(zip(a.keep, b.keep)):
                if ta.dtype == torch.float16:
                    assert_close(to_host(tb.float()), to_host(ta.float()), what=f"step {pos} tensor {i}")
                elif ta.dtype == torch.float32 and ta.numel() < 5_000_000:
                    assert_close(to_host(tb), to_host(ta), rel=1e-3, max_abs=2e-2, what=f"step {pos} tensor {i}")
    finally:
        a.close()
        b.close()


@_PROJ_OFF
def test_complete_layers_persistent_greedy_08b_shape(anelm, orc, dev):
    """Greedy decoding through the persistent complete step at the
    reference's default Qwen3.5-0.8B shape (hidden 1024, inter 3584, 8 q /
    2 kv heads, 16 DeltaNet heads), four layers: two independent loops, 32
    tokens, identical (the seed's smallest top-2 gap is checked first)."""
    m = tiny_lm(2048, dims=_DIMS_08B)
    ref = OracleLM(orc, m)
    want, gaps, tok = [], [], 1
    for pos in range(32):
        _, logits = ref.step(tok, pos)
        tok, adj = orc.sample_token(logits, np.array(want, np.int32), 0.0, 1.2, 256, 0.1, 0.5)
        top2 = np.sort(adj)[-2:]
        gaps.append(float(top2[1] - top2[0]))
        want.append(tok)
    assert min(gaps) > 1e-3, "seeded model has a near-tie: pick another seed"
    gpu = _persistent_lm(anelm, m, dev)
    got, tok = [], 1
    try:
        for pos in range(32):
            logits = gpu.forward(tok)
            rec = to_dev(np.array(got, np.int32), dev) if got else None
            tok = int(to_host(anelm.ops.sample_token(logits, rec, 0.0, 1.2, 256, 0.1, 0.5))[0])
            got.append(tok)
    finally:
        gpu.close()
    assert got == want, next(i for i, (a, b) in enumerate(zip(got, want)) if a != b)


def test_complete_step_graph_replays(anelm, dev):
    """GRAPH mode captures the complete layers once (on a side stream: capture
    needs a non-null stream); every replay from the same inputs gives the
    eager step's hidden state (the conv ring, states and KV slot a replay
    writes are restored between replays, with eager work in between)."""
    m = tiny_lm(2029)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        eager = StepLM(anelm, m, dev, mode=anelm.STEP_EAGER)
        try:
            eager.x.copy_(eager.embed[5])
            anelm.call("anelm_hybrid_step_run", eager.handle, eager.stream)
            want = to_host(eager.x)
        finally:
            eager.close()
        g = StepLM(anelm, m, dev, mode=anelm.STEP_GRAPH)
        try:
            snap = [t.clone() for t in g.keep]
            first = None
            for rep in range(3):
                for t, s0 in zip(g.keep, snap):
                    t.copy_(s0)
                g.x.copy_(g.embed[5])
                anelm.call("anelm_hybrid_step_run", g.handle, g.stream)
                got = to_host(g.x)
                assert_close(got, want, rel=1e-6, max_abs=1e-5, what=f"replay {rep} vs eager")
                if first is None:
                    first = got
                assert np.array_equal(got, first), f"replay {rep} differs from replay 0"
        finally:
            g.close()
