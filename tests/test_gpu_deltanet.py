"""GPU parity of the Gated-DeltaNet kernels against the oracle: the decode
step for all heads (both update orders, gated-norm epilogue) and the prefill
over many tokens (output rows and final state)."""
import numpy as np
import pytest

from gpu_util import assert_close, to_dev, to_host
from workloads import deltanet_case

pytestmark = pytest.mark.gpu


def _dev_case(c, dev):
    return {k: to_dev(getattr(c, k), dev) for k in ("state", "q", "k", "v", "a", "b", "A",
                                                     "dt_bias", "z", "norm_w")}


@pytest.mark.parametrize("Hk,Hv,flags", [
    (16, 16, 1),      # 16 heads, the DeltaNet decode workload
    (16, 16, 3),      # transformers (decay-first) order
    (16, 32, 1),      # 4B layer: 16 key / 32 value heads
    (16, 32, 5),      # with the rmsnorm_gated epilogue
    (4, 32, 7),
    (16, 16, 0),      # inputs used as given (no l2 norm)
])
def test_deltanet_decode(anelm, orc, dev, Hk, Hv, flags):
    c = deltanet_case(500 + Hv + flags, Hk=Hk, Hv=Hv)
    d = _dev_case(c, dev)
    y = anelm.ops.deltanet_decode(d["state"], d["q"], d["k"], d["v"], d["a"], d["b"], d["A"],
                                  d["dt_bias"], flags, d["z"], d["norm_w"])
    yw, Sw = orc.deltanet_decode(c.state, c.q, c.k, c.v, c.a, c.b, c.A, c.dt_bias, flags, c.z,
                                 c.norm_w)
    assert_close(to_host(y), yw, what="y")
    assert_close(to_host(d["state"]), Sw, what="state")


def test_deltanet_decode_repeated_steps(anelm, orc, dev):
    """Ten steps in a row; the epilogue counter is reused across calls."""
    c = deltanet_case(510, Hk=16, Hv=32)
    d = _dev_case(c, dev)
    S = c.state
    rng = np.random.default_rng(511)
    for _ in range(10):
        q = rng.standard_normal((16, 128)).astype(np.float32)
        k = rng.standard_normal((16, 128)).astype(np.float32)
        v = rng.standard_normal((32, 128)).astype(np.float32)
        a = rng.standard_normal(32).astype(np.float32)
        b = rng.standard_normal(32).astype(np.float32)
        y = anelm.ops.deltanet_decode(d["state"], to_dev(q, dev), to_dev(k, dev), to_dev(v, dev),
                                      to_dev(a, dev), to_dev(b, dev), d["A"], d["dt_bias"], 5,
                                      d["z"], d["norm_w"])
        yw, S = orc.deltanet_decode(S, q, k, v, a, b, c.A, c.dt_bias, 5, c.z, c.norm_w)
        assert_close(to_host(y), yw)
    assert_close(to_host(d["state"]), S)


@pytest.mark.parametrize("S,Hk,Hv,flags", [(1, 2, 4, 1), (37, 4, 8, 1), (300, 2, 4, 3),
                                           (512, 16, 32, 1)])
def test_deltanet_prefill(anelm, orc, dev, S, Hk, Hv, flags):
    c = deltanet_case(520 + S, Hk=Hk, Hv=Hv, S=S)
    d = _dev_case(c, dev)
    y = anelm.ops.deltanet_prefill(d["state"], d["q"], d["k"], d["v"], d["a"], d["b"], d["A"],
                                   d["dt_bias"], flags)
    yw, Sw = orc.deltanet_prefill(c.state, c.q, c.k, c.v, c.a, c.b, c.A, c.dt_bias, flags)
    assert_close(to_host(y), yw, what="y")
    assert_close(to_host(d["state"]), Sw, what="state")


def test_deltanet_prefill_matches_decode_chain(anelm, dev):
    """Prefill over S tokens == S decode steps, both on the GPU."""
    c = deltanet_case(530, Hk=4, Hv=8, S=20)
    d = _dev_case(c, dev)
    y = to_host(anelm.ops.deltanet_prefill(d["state"], d["q"], d["k"], d["v"], d["a"], d["b"],
                                           d["A"], d["dt_bias"], 1))
    d2 = _dev_case(c, dev)
    for t in range(20):
        yt = anelm.ops.deltanet_decode(d2["state"], d2["q"][t].contiguous(), d2["k"][t].contiguous(),
                                       d2["v"][t].contiguous(), d2["a"][t].contiguous(),
                                       d2["b"][t].contiguous(), d2["A"], d2["dt_bias"], 1)
        assert_close(to_host(yt), y[t], rel=1e-5, max_abs=1e-4)
    assert_close(to_host(d2["state"]), to_host(d["state"]), rel=1e-5, max_abs=1e-4)


@pytest.mark.parametrize("S,flags", [(64, 1), (65, 3), (200, 1)])
def test_deltanet_prefill_scan_path(anelm, orc, dev, S, flags):
    """chunk=1 selects the token-by-token scan; it matches the oracle too."""
    c = deltanet_case(560 + S, Hk=4, Hv=8, S=S)
    d = _dev_case(c, dev)
    y = anelm.ops.deltanet_prefill(d["state"], d["q"], d["k"], d["v"], d["a"], d["b"], d["A"],
                                   d["dt_bias"], flags, chunk=1)
    yw, Sw = orc.deltanet_prefill(c.state, c.q, c.k, c.v, c.a, c.b, c.A, c.dt_bias, flags)
    assert_close(to_host(y), yw, what="y")
    assert_close(to_host(d["state"]), Sw, what="state")


@pytest.mark.parametrize("flags", [1, 3])
def test_deltanet_prefill_chunked_matches_scan_4096(anelm, dev, flags):
    """The prefill workload size (4096 tokens, 16 key / 32 value heads): the
    chunked form (64-token chunks) against the token-by-token scan, both on the
    GPU (the sequential oracle at this size takes minutes)."""
    c = deltanet_case(570 + flags, Hk=16, Hv=32, S=4096)
    d = _dev_case(c, dev)
    y = to_host(anelm.ops.deltanet_prefill(d["state"], d["q"], d["k"], d["v"], d["a"], d["b"], d["A"],
                                           d["dt_bias"], flags))
    d2 = _dev_case(c, dev)
    y2 = to_host(anelm.ops.deltanet_prefill(d2["state"], d2["q"], d2["k"], d2["v"], d2["a"], d2["b"],
                                            d2["A"], d2["dt_bias"], flags, chunk=1))
    assert_close(y, y2, rel=1e-4, max_abs=1e-3, what="y")
    assert_close(to_host(d["state"]), to_host(d2["state"]), rel=1e-4, max_abs=1e-3, what="state")


@pytest.mark.parametrize("flags", [1, 3])
def test_deltanet_prefill_4096_matches_oracle_on_head_subsets(anelm, orc, dev, flags):
    """The prefill workload at full size (4096 tokens, 16 key / 32 value
    heads, chunked form) against the oracle's sequential recurrence on
    subsets of heads: value heads are independent given their key head
    (qwen3_5.cpp:890 maps value head h to key head h / 2 here), so the oracle
    runs value heads (2kh, 2kh + 1) with key head kh alone -- the same
    per-head arithmetic as the full run -- for kh = 0, 7 and 15, in both
    orders (cpu_ops and decay-first)."""
    c = deltanet_case(590 + flags, Hk=16, Hv=32, S=4096)
    d = _dev_case(c, dev)
    print(f"deltanet prefill 4096 x 16k/32v flags {flags}", flush=True)
    y = to_host(anelm.ops.deltanet_prefill(d["state"], d["q"], d["k"], d["v"], d["a"], d["b"], d["A"],
                                           d["dt_bias"], flags))
    st = to_host(d["state"])
    for kh in (0, 7, 15):
        vs = [2 * kh, 2 * kh + 1]
        yw, Sw = orc.deltanet_prefill(c.state[vs], c.q[:, kh:kh + 1], c.k[:, kh:kh + 1], c.v[:, vs],
                                      c.a[:, vs], c.b[:, vs], c.A[vs], c.dt_bias[vs], flags)
        assert_close(y[:, vs], yw, what=f"y of value heads {vs}")
        assert_close(st[vs], Sw, what=f"state of value heads {vs}")


def test_deltanet_prefill_rejects_other_chunks(anelm, dev):
    c = deltanet_case(580, Hk=2, Hv=4, S=8)
    d = _dev_case(c, dev)
    with pytest.raises(anelm.AnelmError):
        anelm.ops.deltanet_prefill(d["state"], d["q"], d["k"], d["v"], d["a"], d["b"], d["A"],
                                   d["dt_bias"], 1, chunk=32)


@pytest.mark.parametrize("Hk,Hv,flags", [
    (16, 32, 5),      # 4B layer as the model runs it: l2 norm, gated norm, 2 value heads per key head
    (16, 16, 5),      # 0.8B layer (one value head per key head)
    (4, 16, 1),       # ungated: 4 column slabs x 4 value heads read each key head's ring
    (16, 32, 7),      # transformers order
])
def test_deltanet_decode_from_proj(anelm, orc, dev, Hk, Hv, flags):
    """Conv ring + SiLU + split + recurrence from the raw first projection
    (qwen3_5.cpp:849-908), six steps in a row so the ring position cycles
    twice; outputs, states and the conv ring are compared every step."""
    import ctypes
    rng = np.random.default_rng(700 + Hk + Hv + flags)
    d, K = 128, 4
    qkv = 2 * Hk * d + Hv * d
    S = (0.1 * rng.standard_normal((Hv, d, d))).astype(np.float32)
    conv_w = (0.5 * rng.standard_normal((qkv, K))).astype(np.float32)
    cs = (0.5 * rng.standard_normal((qkv, K - 1))).astype(np.float32)
    A = np.exp(rng.uniform(0, np.log(16), Hv)).astype(np.float32)
    dtb = rng.standard_normal(Hv).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    Sd, csd = to_dev(S, dev), to_dev(cs, dev)
    cwd, Ad, dtd, nwd = (to_dev(a, dev) for a in (conv_w, A, dtb, nw))
    pos_ref, pos_gpu = 1, ctypes.c_int(1)
    for t in range(6):
        proj = rng.standard_normal(qkv + Hv * d + 2 * Hv).astype(np.float32)
        y = anelm.ops.deltanet_decode_from_proj(Sd, csd, pos_gpu, to_dev(proj, dev), cwd, Ad, dtd,
                                                nwd if flags & 4 else None, Hk, flags, K)
        yw, S, cs, pos_ref = orc.deltanet_from_proj(S, cs, pos_ref, proj, conv_w, A, dtb, nw, Hk, Hv,
                                                    K, flags)
        assert pos_gpu.value == pos_ref
        assert_close(to_host(y), yw, what=f"y step {t}")
        assert_close(to_host(Sd), S, what=f"state step {t}")
        assert np.array_equal(to_host(csd), cs), f"conv ring step {t}"
