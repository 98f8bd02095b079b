"""GPU parity of the attention kernels against the oracle:
gqa_attention over fp16/fp32 ring caches, the fused full-attention decode step
(norms + RoPE + append + attention + gate), paged batched decode and causal
prefill."""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, to_dev, to_host
from workloads import attn_decode_case, f16, prefill_inputs, widen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nh,nkv,D,start,length,cap", [
    (8, 2, 256, 0, 513, 2048),       # 0.8B-shaped
    (16, 4, 256, 1900, 700, 2048),   # ring wrap
    (16, 2, 128, 0, 3000, 4096),     # G = 8
    (4, 4, 64, 3, 1, 16),            # one key
    (2, 2, 64, 10, 64, 64),          # full ring
    (16, 4, 256, 0, 8192, 8192),     # 4B-shaped context
])
@pytest.mark.parametrize("kv16", [True, False])
def test_gqa_attention(anelm, orc, dev, nh, nkv, D, start, length, cap, kv16):
    rng = np.random.default_rng(200 + length)
    q = rng.standard_normal((nh, 2 * D)).astype(np.float32)
    kc16 = f16(rng.standard_normal((cap, nkv, D)))
    vc16 = f16(rng.standard_normal((cap, nkv, D)))
    kc, vc = widen(kc16), widen(vc16)
    want = orc.gqa_attention(q, kc, vc, nh, nkv, D, 2 * D, start, length, cap)
    dk = to_dev(kc16 if kv16 else kc, dev)
    dv = to_dev(vc16 if kv16 else vc, dev)
    got = anelm.ops.gqa_attention(to_dev(q, dev), dk, dv, nh, nkv, D, 2 * D, start, length, cap)
    assert_close(to_host(got), want, what=f"gqa {nh}/{nkv} D{D} len{length}")


def test_gqa_attention_empty_cache(anelm, dev):
    out = torch.full((8, 256), 7.0, device=dev)
    q = torch.zeros(8, 512, device=dev)
    kc = torch.zeros(4, 2, 256, device=dev, dtype=torch.float16)
    anelm.ops.gqa_attention(q, kc, kc, 8, 2, 256, 512, 0, 0, 4, out=out)
    assert torch.all(out == 0)


def _run_decode(anelm, c, dev, rope_mode=0, gate=True, cos_row=None, sin_row=None):
    dk, dv = to_dev(c.k_cache, dev), to_dev(c.v_cache, dev)
    ring = anelm.ops.KVRing(c.capacity, c.start, c.length)
    out = anelm.ops.full_attn_decode(
        to_dev(c.q_gate, dev), to_dev(c.k, dev), to_dev(c.v, dev), dk, dv, to_dev(c.q_norm_w, dev),
        to_dev(c.k_norm_w, dev), ring, c.n_heads, c.n_kv_heads, c.head_dim, c.rot_dim, c.pos,
        c.theta, c.eps, rope_mode, gate, cos_row, sin_row)
    return to_host(out), to_host(dk), to_host(dv), ring.start.value, ring.len.value


def _oracle_decode(orc, c, rope_mode=0, gate=True):
    return orc.full_attn_decode(c.q_gate, c.k, c.v, c.k_cache, c.v_cache, c.q_norm_w, c.k_norm_w,
                                c.n_heads, c.n_kv_heads, c.head_dim, c.rot_dim, c.pos, c.theta,
                                c.eps, rope_mode, gate, c.start, c.length, c.capacity)


def _check_decode(got, want):
    out, kc, vc, st, ln = got
    wo, wk, wv, wst, wln = want
    assert (st, ln) == (wst, wln)
    assert_close(out, wo, what="decode out")
    # the appended rows agree to one fp16 ulp (normalisation sums differ in
    # order); every other slot is untouched
    dk = np.abs(kc.astype(np.int32) - wk.astype(np.int32))
    assert dk.max() <= 1 and np.count_nonzero(dk) <= 8
    assert np.array_equal(vc, wv)


def test_full_attn_decode_08b_step(anelm, orc, dev):
    """0.8B-shaped step: 8 q / 2 kv heads, D 256, 512 cached, position 512."""
    c = attn_decode_case(300)
    _check_decode(_run_decode(anelm, c, dev), _oracle_decode(orc, c))


def test_full_attn_decode_4b_step(anelm, orc, dev):
    """4B-shaped step: 16 q / 4 kv heads over 8191 cached keys -> 8192."""
    c = attn_decode_case(301, n_heads=16, n_kv_heads=4, cached=8191, capacity=8192, pos=8191)
    _check_decode(_run_decode(anelm, c, dev), _oracle_decode(orc, c))


@pytest.mark.parametrize("rope_mode,gate", [(1, True), (0, False), (1, False)])
def test_full_attn_decode_variants(anelm, orc, dev, rope_mode, gate):
    c = attn_decode_case(302 + rope_mode, n_heads=16, n_kv_heads=4, cached=777, capacity=1024,
                         start=900)
    _check_decode(_run_decode(anelm, c, dev, rope_mode, gate), _oracle_decode(orc, c, rope_mode, gate))


@pytest.mark.parametrize("n_heads,n_kv_heads,head_dim,cached", [
    (8, 2, 256, 127),    # G 4, 64-key splits: 2 splits, the smallest in-kernel merge
    (8, 2, 256, 1023),   # 16 splits, the largest merged in the split kernel
    (8, 2, 256, 1024),   # 17 splits: the merge kernel
    (16, 2, 128, 300),   # G 8, 32-key splits: 10 splits
    (4, 2, 128, 700),    # G 2, 128-key splits (workgroup-wide softmax): 6 splits
    (4, 4, 64, 1000),    # G 1, 256-key splits: 4 splits
])
def test_full_attn_decode_split_merge(anelm, orc, dev, n_heads, n_kv_heads, head_dim, cached):
    """Split counts around the in-kernel merge of the split records (up to 16
    splits of 256/G keys merged by the last workgroup of each kv head, more by
    a second kernel) and the other head groupings, over a wrapped ring,
    against the oracle."""
    c = attn_decode_case(330 + cached % 97, n_heads=n_heads, n_kv_heads=n_kv_heads, head_dim=head_dim,
                         cached=cached, capacity=cached + 5, start=7)
    _check_decode(_run_decode(anelm, c, dev), _oracle_decode(orc, c))


def test_full_attn_decode_table_row(anelm, orc, dev):
    """cos/sin passed as the reference's table row give the same step."""
    c = attn_decode_case(305)
    cs, sn = orc.rope_table(c.pos + 1, c.rot_dim, c.theta)
    _check_decode(_run_decode(anelm, c, dev, cos_row=cs[c.pos], sin_row=sn[c.pos]),
                  _oracle_decode(orc, c))


def test_full_attn_decode_consecutive_steps_wrap_ring(anelm, orc, dev):
    """Five steps through a small full ring: slots are overwritten oldest first."""
    rng = np.random.default_rng(306)
    c = attn_decode_case(306, n_heads=8, n_kv_heads=2, cached=30, capacity=32, start=0)
    dk, dv = to_dev(c.k_cache, dev), to_dev(c.v_cache, dev)
    ring = anelm.ops.KVRing(c.capacity, c.start, c.length)
    kc, vc, st, ln = c.k_cache, c.v_cache, c.start, c.length
    qn, kn = to_dev(c.q_norm_w, dev), to_dev(c.k_norm_w, dev)
    for step in range(5):
        qg = rng.standard_normal((8, 512)).astype(np.float32)
        k = rng.standard_normal((2, 256)).astype(np.float32)
        v = rng.standard_normal((2, 256)).astype(np.float32)
        pos = 30 + step
        out = anelm.ops.full_attn_decode(to_dev(qg, dev), to_dev(k, dev), to_dev(v, dev), dk, dv,
                                         qn, kn, ring, 8, 2, 256, 64, pos)
        wo, kc, vc, st, ln = orc.full_attn_decode(qg, k, v, kc, vc, c.q_norm_w, c.k_norm_w, 8, 2,
                                                  256, 64, pos, 1e7, 1e-6, 0, True, st, ln, 32)
        assert (ring.start.value, ring.len.value) == (st, ln)
        assert_close(to_host(out), wo, what=f"step {step}")
        kc = to_host(dk)   # continue from the device cache (fp16 ulp differences stay local)
    assert (st, ln) == (3, 32)


@pytest.mark.parametrize("nh,nkv,D,P", [(16, 4, 256, 16), (16, 2, 128, 5), (4, 4, 64, 32), (8, 1, 128, 1)])
def test_paged_decode(anelm, orc, dev, nh, nkv, D, P):
    """Ragged sequences over shuffled pages (lengths cross the split sizes of
    every head grouping; page sizes that do and do not divide a split)."""
    rng = np.random.default_rng(307 + P)
    n_seqs = 6
    lens = np.array([1, 17, 300, 1024, 2049, 0], np.int32)
    max_len = 2049
    max_pages = (max_len + P - 1) // P
    n_pages = int(sum((l + P - 1) // P for l in lens)) + 3
    perm = rng.permutation(n_pages)
    table = np.zeros((n_seqs, max_pages), np.int32)
    kp16 = f16(rng.standard_normal((n_pages, nkv, P, D)))
    vp16 = f16(rng.standard_normal((n_pages, nkv, P, D)))
    q = rng.standard_normal((n_seqs, nh, D)).astype(np.float32)
    used = 0
    for s, l in enumerate(lens):
        npg = (l + P - 1) // P
        table[s, :npg] = perm[used:used + npg]
        used += npg
    got = to_host(anelm.ops.attn_decode_paged(
        to_dev(q, dev), to_dev(kp16, dev), to_dev(vp16, dev), to_dev(table, dev), to_dev(lens, dev),
        max_len, nh, nkv, D, P))
    for s, l in enumerate(lens):
        if l == 0:
            assert np.all(got[s] == 0)
            continue
        pages = table[s, :(l + P - 1) // P]
        kc = widen(kp16[pages]).transpose(0, 2, 1, 3).reshape(-1, nkv, D)[:l]
        vc = widen(vp16[pages]).transpose(0, 2, 1, 3).reshape(-1, nkv, D)[:l]
        want = orc.gqa_attention(q[s], kc, vc, nh, nkv, D, D, 0, l, l)
        assert_close(got[s], want, what=f"seq {s} len {l}")


# ---------------------------------------------------------------- prefill
@pytest.mark.parametrize("S,Hq,Hkv,D", [(100, 4, 1, 256), (77, 8, 2, 128), (64, 2, 2, 256),
                                        (130, 16, 2, 128), (1, 4, 1, 256), (95, 8, 2, 256),
                                        (257, 16, 4, 256)])
def test_prefill_small(anelm, orc, dev, S, Hq, Hkv, D):
    q, k, v = prefill_inputs(400 + S, S, Hq, Hkv, D)
    got = to_host(anelm.ops.attn_prefill(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev)))
    assert_close(got, orc.prefill_attention(q, k, v), what=f"prefill S{S} {Hq}/{Hkv} D{D}")


def test_prefill_4096_rows(anelm, orc, dev):
    """Causal prefill at S=4096, 16 q / 4 kv heads, D 256: sampled rows vs the
    oracle (the oracle runs each row as a decode call over keys 0..t)."""
    S, Hq, Hkv, D = 4096, 16, 4, 256
    q, k, v = prefill_inputs(401, S, Hq, Hkv, D)
    out = anelm.ops.attn_prefill(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev))
    got = to_host(out)
    rows = [0, 1, 31, 32, 33, 63, 64, 127, 128, 1000, 2047, 2048, 3071, 4094, 4095]
    rows += list(np.random.default_rng(402).integers(0, S, 5))
    for t in rows:
        want = orc.prefill_attention(q, k, v, int(t), int(t) + 1)[0]
        assert_close(got[t], want, what=f"row {t}")
    # fp16 output variant: same values rounded
    got16 = widen(to_host(anelm.ops.attn_prefill(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev),
                                                 torch.float16)))
    assert_close(got16, got, what="fp16 output")


def test_prefill_repeated_calls_are_identical(anelm, orc, dev):
    """Split blocks are merged through per-call counters that each call leaves
    zeroed: back-to-back calls of different sizes (odd block count, middle
    unit, split pairs) give bit-identical rows, and match the oracle."""
    runs = {}
    for S in (700, 130, 700, 64, 700):
        q, k, v = prefill_inputs(990 + S, S, 16, 4, 256)
        got = to_host(anelm.ops.attn_prefill(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev)))
        if S in runs:
            assert np.array_equal(got, runs[S]), f"S={S}: repeated call differs"
        else:
            runs[S] = got
            for t in (0, S // 3, S - 1):
                assert_close(got[t], orc.prefill_attention(q, k, v, t, t + 1)[0], what=f"S{S} row {t}")


def test_full_attn_decode_without_norms(anelm, orc, dev):
    """q/k arriving normalised (scripts/serve_hybrid.py:89-107: half-split RoPE,
    cache append, attention, sigmoid gate, no q/k RMSNorm): NULL norm weights,
    checked against the oracle's RoPE, fp16 append and gqa_attention."""
    c = attn_decode_case(321, n_heads=16, n_kv_heads=4, head_dim=256, cached=300, capacity=4096)
    D, G = c.head_dim, c.n_heads
    dk, dv = to_dev(c.k_cache, dev), to_dev(c.v_cache, dev)
    ring = anelm.ops.KVRing(c.capacity, c.start, c.length)
    out = anelm.ops.full_attn_decode(to_dev(c.q_gate, dev), to_dev(c.k, dev), to_dev(c.v, dev), dk, dv,
                                     None, None, ring, G, c.n_kv_heads, D, c.rot_dim, c.pos, c.theta,
                                     c.eps, rope_mode=1, gate=True)
    q, k = orc.apply_rope(c.q_gate, c.k, G, c.n_kv_heads, D, 2 * D, D, c.rot_dim, c.pos, c.theta, mode=1)
    slot = (c.start + c.length) % c.capacity
    kc, vc = c.k_cache.copy(), c.v_cache.copy()
    kc[slot], vc[slot] = f16(k), f16(c.v)
    want = orc.gqa_attention(q, widen(kc), widen(vc), G, c.n_kv_heads, D, 2 * D, c.start, c.length + 1,
                             c.capacity)
    want = orc.mul_sigmoid(want, c.q_gate[:, D:])
    assert (ring.start.value, ring.len.value) == (c.start, c.length + 1)
    assert_close(to_host(out), want, what="decode without norms")
    assert np.array_equal(to_host(dk)[slot], kc[slot]) and np.array_equal(to_host(dv)[slot], vc[slot])
