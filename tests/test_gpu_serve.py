"""The serve_hybrid.py CPU-attention swap (scripts/serve_hybrid.py:85-132)
executed: ane_lm_amd.serve_hybrid.cpu_attention -- same name, arguments and
result as the reference function -- over device head-major caches, against
the oracle's composition of the same steps, for a run of decode positions
from an empty cache and for one step deep into a filled one."""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, to_dev, to_host
from workloads import f16, oracle_serve_attention, widen

pytestmark = pytest.mark.gpu


def _inputs(rng, sh):
    return f16(rng.standard_normal(sh))


def test_cpu_attention_decode_run(anelm, orc, dev):
    """Positions 0..47 from empty fp32 caches, host numpy fp16 in and out, as
    serve_hybrid.py's decode loop calls it (:242-272)."""
    from ane_lm_amd import serve_hybrid as sh
    rng = np.random.default_rng(1200)
    caches = sh.make_kv_caches(2, device=dev)
    kc = np.zeros((4, sh.CONTEXT, 256), np.float32)
    vc = np.zeros_like(kc)
    for pos in range(48):
        qg, k, v = _inputs(rng, (1, 16 * 512)), _inputs(rng, (1, 4 * 256)), _inputs(rng, (1, 4 * 256))
        got = sh.cpu_attention(qg.view(np.float16), k.view(np.float16), v.view(np.float16), pos, caches, 1)
        want = oracle_serve_attention(orc, qg, k, v, pos, kc, vc, sh.ROPE_COS[pos], sh.ROPE_SIN[pos])
        assert got.dtype == np.float16 and got.shape == (1, sh.ATTN_DIM)
        assert_close(widen(got.view(np.uint16)), widen(want), what=f"pos {pos}")
    # the layer's caches hold the rotated keys and the values, other layers untouched
    assert np.array_equal(to_host(caches[1][0])[:, :48], kc[:, :48])
    assert np.array_equal(to_host(caches[1][1])[:, :48], vc[:, :48])
    assert not torch.any(caches[0][0]).item()


@pytest.mark.parametrize("cache_dtype", [torch.float32, torch.float16])
def test_cpu_attention_deep_position(anelm, orc, dev, cache_dtype):
    """One step at position 3000 of a filled cache, device fp16 tensors in
    and out; an fp16 cache holds the fp16 rounding of the same values."""
    from ane_lm_amd import serve_hybrid as sh
    rng = np.random.default_rng(1201 + (cache_dtype == torch.float16))
    pos = 3000
    kc = rng.standard_normal((4, sh.CONTEXT, 256)).astype(np.float32)
    vc = rng.standard_normal((4, sh.CONTEXT, 256)).astype(np.float32)
    if cache_dtype == torch.float16:
        kc, vc = widen(f16(kc)), widen(f16(vc))
    caches = [(to_dev(kc, dev).to(cache_dtype), to_dev(vc, dev).to(cache_dtype))]
    qg, k, v = _inputs(rng, (1, 16 * 512)), _inputs(rng, (1, 4 * 256)), _inputs(rng, (1, 4 * 256))
    got = sh.cpu_attention(to_dev(qg, dev), to_dev(k, dev), to_dev(v, dev), pos, caches, 0)
    assert got.is_cuda and got.dtype == torch.float16
    want = oracle_serve_attention(orc, qg, k, v, pos, kc, vc, sh.ROPE_COS[pos], sh.ROPE_SIN[pos],
                                  kv_f16=cache_dtype == torch.float16)
    assert_close(widen(to_host(got)), widen(want), what=f"pos {pos} {cache_dtype}")
