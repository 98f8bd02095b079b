"""GPU parity of the batched decode step executor (anelm_batch_step_*):
32 sequences at the Qwen3.5-4B shape through 4 hybrid layers (3 DeltaNet
launches over 32 x 32 = 1024 value heads, 1 fused paged-attention layer over
ragged shuffled pages), the batched LUT6 FFN, the final norm and the LM-head
top-k, two advancing steps, against the oracle per sequence."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import assert_close, to_dev, to_host
from workloads import OracleBatch, batch_model, lut6_matrix, widen

pytestmark = pytest.mark.gpu

_P = ctypes.c_void_p


class DeviceBatch:
    def __init__(self, anelm, m, dev, lm=None, top_k=4, final_norm=None, rope_rows=4096):
        d = m.dims
        B = len(m.lens)
        self.keep = []
        self.outs = []
        self.layers = (anelm.BatchLayer * len(m.layers))()
        ptr = lambda t: t.data_ptr()
        max_pages = 1
        for i, L in enumerate(m.layers):
            t = {}
            D = self.layers[i]
            D.kind = L["kind"]
            for k, v in L.items():
                if isinstance(v, np.ndarray):
                    t[k] = to_dev(v, dev)
            if L["kind"] == 1:
                c = L["pages"]
                t["k_pages"], t["v_pages"] = to_dev(c.k_pages, dev), to_dev(c.v_pages, dev)
                t["page_table"] = to_dev(c.table, dev)
                max_pages = c.table.shape[1]
                self.n_pages, self.page_size = c.k_pages.shape[0], c.page_size
                out_len = d["n_heads"] * d["head_dim"]
            else:
                D.dn_flags = L["dn_flags"]
                out_len = d["lin_v_heads"] * d["lin_dim"]
            t["core_out"] = torch.zeros(B, out_len, device=dev)
            for k, v in t.items():
                setattr(D, k, ptr(v))
            self.keep.append(t)
            self.outs.append(t["core_out"])
        self.x = to_dev(m.x, dev)
        self.lens = to_dev(m.lens, dev)
        self.rope = anelm.ops.rope_table(d["rot_dim"], rope_rows, d["theta"], dev)
        self.seqs = anelm.BatchSeqs()
        q = self.seqs
        q.n_seqs, q.seq_lens, q.positions = B, ptr(self.lens), None
        q.page_size, q.n_pages, q.max_pages = self.page_size, self.n_pages, max_pages
        q.max_seq_len = max_pages * self.page_size
        q.rope_table, q.rope_rows = ptr(self.rope), rope_rows
        if lm is not None:
            self.lm = (to_dev(lm[0], dev), to_dev(lm[1], dev))
            self.fn = to_dev(final_norm, dev)
            self.top_idx = torch.empty(B, top_k, dtype=torch.int32, device=dev)
            self.top_val = torch.empty(B, top_k, device=dev)
            q.final_norm_w, q.lm_w, q.lm_lut = ptr(self.fn), ptr(self.lm[0]), ptr(self.lm[1])
            q.vocab, q.top_k = lm[1].shape[0] * 32, top_k
            q.top_idx, q.top_val = ptr(self.top_idx), ptr(self.top_val)
        self.dims = anelm.HybridDims(d["hidden"], d["inter"], d["n_heads"], d["n_kv_heads"], d["head_dim"],
                                     d["rot_dim"], 0, d["theta"], d["eps"], d["lin_k_heads"],
                                     d["lin_v_heads"], d["lin_dim"])


def test_batch_step_32_sequences_matches_oracle(anelm, orc, dev):
    m = batch_model(1300, 4, 32, lut_std=0.005)
    V, k = 8192, 4
    lm_w, lm_lut, _ = lut6_matrix(1301, V, m.dims["hidden"])
    fnorm = (1 + 0.02 * np.random.default_rng(1302).standard_normal(m.dims["hidden"])).astype(np.float32)
    db = DeviceBatch(anelm, m, dev, lm=(lm_w, lm_lut), top_k=k, final_norm=fnorm)
    h = _P()
    rc = anelm.status("anelm_batch_step_create", ctypes.byref(h), ctypes.byref(db.dims), db.layers,
                      len(m.layers), ctypes.byref(db.seqs), _P(db.x.data_ptr()))
    assert rc == 0, anelm.last_error()
    ob = OracleBatch(orc, m, steps=2)
    exact_rows = 0
    try:
        for step in range(2):
            print(f"batch step {step}: 32 sequences, 4 layers", flush=True)
            anelm.call("anelm_batch_step_run", h, 1, _P(torch.cuda.current_stream().cuda_stream))
            torch.cuda.synchronize()
            outs = ob.step()
            for i, L in enumerate(m.layers):
                got = to_host(db.outs[i])
                for s in range(32):
                    assert_close(got[s], outs[i][s], what=f"step {step} layer {i} seq {s} core output")
                if L["kind"] == 0:
                    st = to_host(db.keep[i]["state"])
                    for s in (0, 13, 31):
                        assert_close(st[s], ob.state[i][s], what=f"step {step} layer {i} seq {s} state")
                else:
                    c = L["pages"]
                    kp = to_host(db.keep[i]["k_pages"])
                    for s in (0, 13, 31):
                        Lk = int(m.lens[s]) + step
                        page, row = c.table[s, Lk // c.page_size], Lk % c.page_size
                        assert_close(widen(kp[page, :, row]), widen(ob.rings[i][s][0][Lk]),
                                     what=f"step {step} layer {i} seq {s} appended k")
            assert_close(to_host(db.x), ob.x, what=f"step {step} hidden states")
            assert np.array_equal(to_host(db.lens), m.lens + step + 1), "seq_lens not advanced"
            # LM head: top-k of the final-normed hidden states
            idx, val = to_host(db.top_idx), to_host(db.top_val)
            for s in range(32):
                xf = orc.rmsnorm(ob.x[s], fnorm, m.dims["eps"])
                logits = orc.lut6_matvec(lm_w, lm_lut, xf, V, m.dims["hidden"])
                oi, ov = orc.topk(logits, k)
                assert_close(val[s], ov, rel=1e-4, max_abs=1e-3, what=f"step {step} seq {s} top values")
                gaps = np.abs(np.diff(np.concatenate([ov, [np.sort(logits)[-k - 1]]])))
                if np.all(gaps > 1e-4 * max(1.0, float(np.abs(ov).max()))):
                    assert np.array_equal(idx[s], oi), f"step {step} seq {s} top indices"
                    exact_rows += 1
        assert exact_rows >= 60, f"only {exact_rows} of 64 rows were separated enough to compare indices"
    finally:
        anelm.call("anelm_batch_step_destroy", h)


def test_batch_step_full_lengths_matches_oracle(anelm, orc, dev):
    """The batched step at the full lengths of the 32-sequence workload:
    lengths U[256, 16384] (sum ~266k keys) over shuffled 16-token pages, so
    the paged attention layer runs its multi-run workgroups and the split
    merge over up to 64 records per (sequence, kv head); 4 layers, one
    advancing step, every core output and the hidden states against the
    oracle per sequence."""
    m = batch_model(1320, 4, 32, lo=256, hi=16384, lut_std=0.005)
    rows = int(m.lens.max()) + 8
    db = DeviceBatch(anelm, m, dev, rope_rows=rows)
    h = _P()
    rc = anelm.status("anelm_batch_step_create", ctypes.byref(h), ctypes.byref(db.dims), db.layers,
                      len(m.layers), ctypes.byref(db.seqs), _P(db.x.data_ptr()))
    assert rc == 0, anelm.last_error()
    try:
        print(f"batch step: 32 sequences, sum of lengths {int(m.lens.sum())}, 4 layers", flush=True)
        anelm.call("anelm_batch_step_run", h, 1, _P(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        ob = OracleBatch(orc, m, steps=1)
        outs = ob.step()
        for i, L in enumerate(m.layers):
            got = to_host(db.outs[i])
            for s in range(32):
                assert_close(got[s], outs[i][s], what=f"layer {i} seq {s} core output (len {int(m.lens[s])})")
        assert_close(to_host(db.x), ob.x, what="hidden states")
        assert np.array_equal(to_host(db.lens), m.lens + 1), "seq_lens not advanced"
    finally:
        anelm.call("anelm_batch_step_destroy", h)


def test_batch_step_stops_at_max_seq_len(anelm, dev):
    """A sequence whose paged cache is full (max_seq_len keys) appends nothing
    (anelm_attn_decode_paged_step): an advancing step leaves its length and
    position where they are and raises the step status; the others advance."""
    m = batch_model(1310, 4, 4, lo=256, hi=300)
    db = DeviceBatch(anelm, m, dev)
    top = int(m.lens.max())
    db.seqs.max_seq_len = top + 1            # the longest sequence fills its cache at step 1
    pos = torch.tensor(m.lens + 1000, dtype=torch.int32, device=dev)
    db.seqs.positions = pos.data_ptr()
    h = _P()
    rc = anelm.status("anelm_batch_step_create", ctypes.byref(h), ctypes.byref(db.dims), db.layers,
                      len(m.layers), ctypes.byref(db.seqs), _P(db.x.data_ptr()))
    assert rc == 0, anelm.last_error()
    st = ctypes.c_int(-1)
    s = _P(torch.cuda.current_stream().cuda_stream)
    try:
        print("batch step at max_seq_len: step 1", flush=True)
        anelm.call("anelm_batch_step_run", h, 1, s)
        anelm.call("anelm_batch_step_status", h, ctypes.byref(st))
        assert st.value == 0
        assert np.array_equal(to_host(db.lens), m.lens + 1)
        print("batch step at max_seq_len: step 2", flush=True)
        anelm.call("anelm_batch_step_run", h, 1, s)
        anelm.call("anelm_batch_step_status", h, ctypes.byref(st))
        assert st.value == 1
        full = m.lens == top
        assert full.any() and not full.all()
        want = np.where(full, m.lens + 1, m.lens + 2)
        assert np.array_equal(to_host(db.lens), want)
        assert np.array_equal(to_host(pos), want + 1000)
        anelm.call("anelm_batch_step_status", h, ctypes.byref(st))
        assert st.value == 0   # cleared by the read
    finally:
        anelm.call("anelm_batch_step_destroy", h)
