"""GPU parity of the row-wise cpu_ops kernels and of the host-pointer compat
tier (include/anelm_cpu_ops.h) against the oracle."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import assert_close, to_dev, to_host

pytestmark = pytest.mark.gpu


def test_rmsnorm_and_gated(anelm, orc, dev):
    rng = np.random.default_rng(100)
    x = rng.standard_normal((12, 256)).astype(np.float32) * 2
    w = (1 + 0.02 * rng.standard_normal(256)).astype(np.float32)
    got = to_host(anelm.ops.rmsnorm(to_dev(x, dev), to_dev(w, dev), 1e-6))
    assert_close(got, orc.rmsnorm(x, w, 1e-6), rel=1e-6, what="rmsnorm")
    z = rng.standard_normal((12, 256)).astype(np.float32)
    got = to_host(anelm.ops.rmsnorm_gated(to_dev(x, dev), to_dev(z, dev), to_dev(w, dev)))
    assert_close(got, orc.rmsnorm_gated(x, z, w), rel=1e-6, what="rmsnorm_gated")


def test_l2norm_activations_softmax_matvec(anelm, orc, dev):
    rng = np.random.default_rng(101)
    x = rng.standard_normal((6, 128)).astype(np.float32) * 3
    t = to_dev(x, dev)
    anelm.ops.l2_normalize_(t)
    assert_close(to_host(t), np.stack([orc.l2_normalize(r) for r in x]), rel=1e-6)
    v = rng.standard_normal(5000).astype(np.float32) * 4
    z = rng.standard_normal(5000).astype(np.float32)
    assert_close(to_host(anelm.ops.silu_(to_dev(v, dev))), orc.silu(v), rel=1e-6)
    assert_close(to_host(anelm.ops.mul_sigmoid_(to_dev(v, dev), to_dev(z, dev))),
                 orc.mul_sigmoid(v, z), rel=1e-6)
    s = (rng.standard_normal((3, 4099)) * 5).astype(np.float32)
    assert_close(to_host(anelm.ops.softmax_(to_dev(s, dev))), np.stack([orc.softmax(r) for r in s]),
                 rel=1e-5)
    W = rng.standard_normal((300, 777)).astype(np.float32)
    xv = rng.standard_normal(777).astype(np.float32)
    assert_close(to_host(anelm.ops.matvec(to_dev(W, dev), to_dev(xv, dev))), orc.matvec(W, xv),
                 rel=1e-5)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("pos", [0, 512, 8191])
def test_rope(anelm, orc, dev, mode, pos):
    rng = np.random.default_rng(102 + pos)
    nq, nkv, D, rot = 16, 4, 256, 64
    q = rng.standard_normal((nq, 2 * D)).astype(np.float32)
    k = rng.standard_normal((nkv, D)).astype(np.float32)
    tq, tk = to_dev(q, dev), to_dev(k, dev)
    anelm.ops.apply_rope_(tq, tk, nq, nkv, D, 2 * D, D, rot, pos, 1e7, mode)
    wq, wk = orc.apply_rope(q, k, nq, nkv, D, 2 * D, D, rot, pos, 1e7, mode=mode)
    # cos/sin come from the same host libm as the oracle: bit-exact
    assert np.array_equal(to_host(tq), wq) and np.array_equal(to_host(tk), wk)
    c, s = orc.rope_table(pos + 1, rot, 1e7)
    tq = to_dev(q, dev)
    anelm.ops.apply_rope_(tq, None, nq, 0, D, 2 * D, D, rot, pos, 1e7, mode, c[pos], s[pos])
    wq, _ = orc.apply_rope(q, k, nq, 0, D, 2 * D, D, rot, pos, 1e7, c[pos], s[pos], mode)
    assert np.array_equal(to_host(tq), wq)


def test_conv1d_update_steps(anelm, orc, dev):
    rng = np.random.default_rng(103)
    C, K = 12352, 4
    w = rng.standard_normal((C, K)).astype(np.float32)
    st_h = np.zeros((C, K - 1), np.float32)
    st_d = to_dev(st_h, dev)
    pos_h, pos_d = 0, ctypes.c_int(0)
    for _ in range(5):
        x = rng.standard_normal(C).astype(np.float32)
        y_h, st_h, pos_h = orc.conv1d_update(st_h, pos_h, x, w, K)
        y_d = anelm.ops.conv1d_update(st_d, pos_d, to_dev(x, dev), to_dev(w, dev), K)
        assert_close(to_host(y_d), y_h, rel=1e-6)
        assert pos_d.value == pos_h
    assert np.array_equal(to_host(st_d), st_h)


@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("dk,dv", [(128, 128), (256, 300), (64, 70)])
def test_ssm_step_single_head(anelm, orc, dev, order, dk, dv):
    """key_dim 256 re-reads its state column in the second pass; 64 and 128 hold it."""
    rng = np.random.default_rng(104 + order + dk)
    S = (0.1 * rng.standard_normal((dk, dv))).astype(np.float32)
    q, k = (rng.standard_normal(dk).astype(np.float32) for _ in range(2))
    v = rng.standard_normal(dv).astype(np.float32)
    tS = to_dev(S, dev)
    y = anelm.ops.ssm_step(tS, to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), 0.9, 0.4,
                           2 if order else 0)
    yw, Sw = orc.ssm_step(S, q, k, v, 0.9, 0.4, order)
    assert_close(to_host(y), yw, rel=1e-5)
    assert_close(to_host(tS), Sw, rel=1e-6)


def _fp(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def test_compat_tier_host_pointers(anelm, orc, dev):
    """The ane_lm:: drop-in (anelm_cpu_*) on host fp32 buffers, synchronous."""
    call = anelm.call
    rng = np.random.default_rng(105)
    x = rng.standard_normal(256).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(256)).astype(np.float32)
    out = np.empty_like(x)
    call("anelm_cpu_rmsnorm", _fp(out), _fp(x), _fp(w), 256, 1e-6)
    assert_close(out, orc.rmsnorm(x, w, 1e-6), rel=1e-6)
    z = rng.standard_normal(256).astype(np.float32)
    call("anelm_cpu_rmsnorm_gated", _fp(out), _fp(x), _fp(z), _fp(w), 256)
    assert_close(out, orc.rmsnorm_gated(x, z, w), rel=1e-6)
    y = x.copy()
    call("anelm_cpu_silu_vec_inplace", _fp(y), 256, None)
    assert_close(y, orc.silu(x), rel=1e-6)
    y = x.copy()
    call("anelm_cpu_mul_sigmoid_inplace", _fp(y), _fp(z), 256, None)
    assert_close(y, orc.mul_sigmoid(x, z), rel=1e-6)
    y = x.copy()
    call("anelm_cpu_softmax", _fp(y), 256)
    assert_close(y, orc.softmax(x), rel=1e-6)
    y = x.copy()
    call("anelm_cpu_l2_normalize", _fp(y), 256)
    assert_close(y, orc.l2_normalize(x), rel=1e-6)
    W = rng.standard_normal((64, 256)).astype(np.float32)
    yv = np.empty(64, np.float32)
    call("anelm_cpu_matvec", _fp(yv), _fp(W), _fp(x), 64, 256)
    assert_close(yv, orc.matvec(W, x), rel=1e-5)
    # apply_rope_cached: q rows of stride 2D, k rows of stride D
    q = rng.standard_normal((8, 512)).astype(np.float32)
    k = rng.standard_normal((2, 256)).astype(np.float32)
    qq, kk = q.copy(), k.copy()
    call("anelm_cpu_apply_rope_cached", _fp(qq), _fp(kk), 8, 2, 256, 512, 256, 64, 300, 1e7, None,
         None)
    wq, wk = orc.apply_rope(q, k, 8, 2, 256, 512, 256, 64, 300, 1e7)
    assert np.array_equal(qq, wq) and np.array_equal(kk, wk)
    # ssm_step
    S = (0.1 * rng.standard_normal((128, 128))).astype(np.float32)
    qs, ks, vs = (rng.standard_normal(128).astype(np.float32) for _ in range(3))
    S2 = S.copy()
    ys = np.empty(128, np.float32)
    call("anelm_cpu_ssm_step", _fp(ys), _fp(S2), _fp(qs), _fp(ks), _fp(vs), 0.8, 0.3, 128, 128)
    yw, Sw = orc.ssm_step(S, qs, ks, vs, 0.8, 0.3, 0)
    assert_close(ys, yw, rel=1e-5)
    assert_close(S2, Sw, rel=1e-6)
    # gqa_attention over an fp32 ring cache, as the reference stores it
    cap = 64
    kc = rng.standard_normal((cap, 2, 256)).astype(np.float32)
    vc = rng.standard_normal((cap, 2, 256)).astype(np.float32)
    o = np.empty((8, 256), np.float32)
    call("anelm_cpu_gqa_attention", _fp(o), _fp(q), _fp(kc), _fp(vc), 8, 2, 256, 512, 50, 40, cap)
    assert_close(o, orc.gqa_attention(q, kc, vc, 8, 2, 256, 512, 50, 40, cap), rel=1e-5)
    call("anelm_cpu_gqa_attention", _fp(o), _fp(q), _fp(kc), _fp(vc), 8, 2, 256, 512, 0, 0, cap)
    assert np.all(o == 0)
    # conv1d_update with its host state_pos
    C, K = 100, 4
    cw = rng.standard_normal((C, K)).astype(np.float32)
    st = np.zeros((C, K - 1), np.float32)
    st_o = st.copy()
    pos = ctypes.c_int(0)
    pos_o = 0
    for _ in range(4):
        xc = rng.standard_normal(C).astype(np.float32)
        yc = np.empty(C, np.float32)
        call("anelm_cpu_conv1d_update", _fp(yc), _fp(st), ctypes.byref(pos), _fp(xc), _fp(cw), C, K)
        yo, st_o, pos_o = orc.conv1d_update(st_o, pos_o, xc, cw, K)
        assert_close(yc, yo, rel=1e-6)
        assert pos.value == pos_o
    assert np.array_equal(st, st_o)
