"""GPU parity of the batched decode over paged fp16 caches at the
32-sequence daemon configuration: the fused per-sequence attention step
(qwen3_5.cpp:944-1002 for every sequence: q/k RMSNorm, RoPE at the
sequence's position, page append, attention, gate) against the oracle's
full_attn_decode on each sequence's gathered pages."""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, to_dev, to_host
from workloads import f16, paged_case, widen

pytestmark = pytest.mark.gpu


def _step_inputs(seed, n, Hq, Hkv, D):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, Hq, 2 * D), dtype=np.float32),
            rng.standard_normal((n, Hkv, D), dtype=np.float32),
            rng.standard_normal((n, Hkv, D), dtype=np.float32),
            (1 + 0.02 * rng.standard_normal(D)).astype(np.float32),
            (1 + 0.02 * rng.standard_normal(D)).astype(np.float32))


def _run_and_check(anelm, orc, dev, c, Hq, Hkv, D, rot, positions=None, table_rows=None, rope_mode=0,
                   norms=True, gate=True, seqs=None, label=""):
    n = len(c.lens)
    qg, k, v, qn, kn = _step_inputs(int(c.lens.sum()) % 1000, n, Hq, Hkv, D)
    kp, vp = to_dev(c.k_pages, dev), to_dev(c.v_pages, dev)
    pos = c.lens if positions is None else np.asarray(positions, np.int32)
    tab = anelm.ops.rope_table(rot, table_rows, 1e7, dev) if table_rows else None
    max_len = int(c.lens.max()) + 1
    out = to_host(anelm.ops.attn_decode_paged_step(
        to_dev(qg, dev), to_dev(k, dev), to_dev(v, dev), kp, vp, to_dev(c.table, dev), to_dev(c.lens, dev),
        to_dev(qn, dev) if norms else None, to_dev(kn, dev) if norms else None, max_len, Hq, Hkv, D,
        c.page_size, rot, rope_mode=rope_mode, gate=gate,
        positions=None if positions is None else to_dev(pos, dev), rope_tab=tab))
    kp_after, vp_after = to_host(kp), to_host(vp)
    # expected pool: the input pages with each sequence's appended row taken
    # from the device (those rows are checked against the oracle below)
    want_k, want_v = c.k_pages.copy(), c.v_pages.copy()
    for s in (range(n) if seqs is None else seqs):
        L = int(c.lens[s])
        kc = f16(c.gather(s, c.k_pages, L + 1))   # capacity L + 1: the append fills the ring
        vc = f16(c.gather(s, c.v_pages, L + 1))
        want, kc2, vc2, st, ln = orc.full_attn_decode(
            qg[s], k[s], v[s], kc, vc, qn if norms else None, kn if norms else None, Hq, Hkv, D, rot,
            int(pos[s]), 1e7, 1e-6, rope_mode, gate, 0, L, L + 1)
        assert (st, ln) == (0, L + 1)
        assert_close(out[s], want, what=f"{label} seq {s} ({L} cached keys, position {pos[s]})")
        page, row = c.table[s, L // c.page_size], L % c.page_size
        for name, got, ref in (("k", kp_after, kc2), ("v", vp_after, vc2)):
            assert_close(widen(got[page, :, row]), widen(ref[L]), what=f"{label} seq {s} appended {name}")
        # v is stored as given: bit-identical to the oracle's rounding
        assert np.array_equal(vp_after[page, :, row], vc2[L]), f"{label} seq {s} appended v bits"
        want_k[page, :, row], want_v[page, :, row] = kp_after[page, :, row], vp_after[page, :, row]
    if seqs is None:
        # every other row of the page pool is untouched
        assert np.array_equal(kp_after, want_k) and np.array_equal(vp_after, want_v), f"{label} page pool"


def test_paged_step_c5(anelm, orc, dev):
    """32 sequences, cached lengths U[256, 16384] (seeded), 16-token shuffled
    pages, 16 q / 4 kv heads, D 256, RoPE rows from the table at each
    sequence's own position."""
    c = paged_case(1200)
    print(f"paged step C5: {len(c.lens)} sequences, {int(c.lens.sum())} cached keys", flush=True)
    _run_and_check(anelm, orc, dev, c, 16, 4, 256, 64, table_rows=16385, label="C5")


def test_paged_step_positions_beyond_table(anelm, orc, dev):
    """Explicit positions, some past the RoPE table (cos / sin evaluated on
    the device there), some with no table at all; lengths crossing split and
    page boundaries (0, 1, a page, a split of 4 chunks)."""
    lens = [0, 1, 15, 16, 255, 256, 257, 1023, 3000]
    c = paged_case(1201, lens=lens)
    positions = [7, 100, 5000, 16, 254, 9000, 257, 1023, 70000]
    _run_and_check(anelm, orc, dev, c, 16, 4, 256, 64, positions=positions, table_rows=2048, label="table+device")
    _run_and_check(anelm, orc, dev, paged_case(1202, lens=lens), 16, 4, 256, 64, positions=positions,
                   label="device RoPE")


@pytest.mark.parametrize("Hq,Hkv,D,P,mode,norms,gate", [(8, 2, 256, 16, 1, True, True),
                                                          (16, 2, 128, 5, 0, False, True),
                                                          (4, 4, 64, 32, 0, True, False),
                                                          (8, 1, 128, 1, 1, True, True)])
def test_paged_step_shapes(anelm, orc, dev, Hq, Hkv, D, P, mode, norms, gate):
    """Head groupings 1-8, head dims 64-256, page sizes 1-32, half-split RoPE,
    no q/k norm (callers with normalised q/k), gate off."""
    c = paged_case(1210 + P, lens=[0, 3, 64, 200, 1100, 2049], Hkv=Hkv, D=D, P=P)
    _run_and_check(anelm, orc, dev, c, Hq, Hkv, D, D // 4, table_rows=4096, rope_mode=mode, norms=norms,
                   gate=gate, label=f"{Hq}q/{Hkv}kv D{D} P{P}")


@pytest.mark.parametrize("mode,rot", [(1, 20), (0, 20), (1, 64), (0, 6)])
def test_paged_step_partial_rotary(anelm, orc, dev, mode, rot):
    """Rotary dims that do not fill whole lanes: half-split pairs whose halves
    straddle lanes (rot_dim 20: the LDS prologue), interleaved pairs ending
    inside a lane (rot_dim 20, 6), and half-split halves of whole lanes
    (rot_dim 64 of D 128)."""
    c = paged_case(1230 + rot + mode, lens=[0, 5, 130, 700, 1500], Hkv=2, D=128, P=16)
    _run_and_check(anelm, orc, dev, c, 8, 2, 128, rot, table_rows=4096, rope_mode=mode,
                   label=f"mode {mode} rot {rot}")


@pytest.mark.parametrize("n_seqs", [2049])
def test_paged_step_many_sequences(anelm, orc, dev, n_seqs):
    """2049 sequences x 8 kv heads (16,392 (sequence, kv head) pairs over the
    resident workgroups' unit shares): most lengths are under 40 keys, every
    97th sequence has 600 (three 256-key splits merged from their records)."""
    rng = np.random.default_rng(1250)
    lens = rng.integers(0, 40, n_seqs)
    lens[::97] = 600
    c = paged_case(1250, lens=lens, Hkv=8, D=64, P=16)
    seqs = sorted(set(range(0, n_seqs, 97)) | set(range(1, 40)) | {n_seqs - 1})
    _run_and_check(anelm, orc, dev, c, 16, 8, 64, 16, table_rows=1024, seqs=seqs, label="merge kernel")
