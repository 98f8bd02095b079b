"""The C ABI from a compiled C++ caller: ane-lm_amd/stream_generate (built by
__graft_entry__.build() from ane-lm_amd/host/stream_generate.cpp) runs the
stream_generate decode loop of generate.cpp:30-140 -- single-token prefill of
the prompt (or the whole prompt through each layer at once), then
sample_token with the generated tokens as the penalty window
-- with every forward on the GPU through anelm_hybrid_step, the LM head and
anelm_sample_token.  Its tokens are compared with the oracle's loop over the
same random-init weights."""
import os
import struct
import subprocess

import numpy as np
import pytest

from workloads import ROOT, OracleLM, tiny_lm

pytestmark = pytest.mark.gpu

BIN = os.path.join(ROOT, "ane-lm_amd", "stream_generate")


def _write_model(m, path):
    """Records (int64 byte count, bytes) in the order the host program reads them."""
    d = m["dims"]
    hdr = struct.pack("<13i2f", d["hidden"], d["inter"], len(m["layers"]), d["n_heads"], d["n_kv_heads"],
                      d["head_dim"], d["rot_dim"], d["lin_k_heads"], d["lin_v_heads"], d["lin_dim"],
                      d["conv_kernel"], d["vocab"], d["cap"], d["theta"], d["eps"])
    with open(path, "wb") as f:
        def rec(b):
            b = b if isinstance(b, bytes) else np.ascontiguousarray(b).tobytes()
            f.write(struct.pack("<q", len(b)))
            f.write(b)
        rec(hdr)
        for L in m["layers"]:
            for key in ("in_norm", "first", "o", "post_norm", "gate", "up", "down"):
                v = L[key]
                if isinstance(v, tuple):
                    rec(v[0])
                    rec(v[1])
                else:
                    rec(v)
            keys = ("q_norm", "k_norm") if L["attn"] else ("conv_w", "A", "dt_bias", "norm_w")
            for key in keys:
                rec(L[key])
        rec(m["embed"])
        rec(m["final_norm"])
        rec(m["lm_head"][0])
        rec(m["lm_head"][1])


def _lcg(seed):
    s = seed
    while True:
        s = (s * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        yield (s >> 11) * (1.0 / 9007199254740992.0)


def _oracle_loop(orc, m, prompt, n, T, seed):
    """generate.cpp:30-140 on the oracle; returns the tokens and, per token,
    the decision margin (top-2 gap of the penalised logits for greedy, the
    distance of the draw from the nearest CDF step when sampling)."""
    ref = OracleLM(orc, m)
    for pos, tok in enumerate(prompt):
        _, logits = ref.step(tok, pos)
    draws = _lcg(seed)
    toks, margins = [], []
    pos = len(prompt)
    for i in range(n):
        r = float(np.float32(next(draws)))
        tok, adj = orc.sample_token(logits, np.array(toks, np.int32), T, 1.2, 256, 0.1, r)
        if T > 0:
            margins.append(float(np.min(np.abs(np.cumsum(adj.astype(np.float64)) - r))))
        else:
            top2 = np.sort(adj)[-2:]
            margins.append(float(top2[1] - top2[0]))
        toks.append(tok)
        if i + 1 < n:
            _, logits = ref.step(tok, pos)
            pos += 1
    return toks, margins


def _run(model, prompt, n, T, seed, prefill_mode=0):
    assert os.path.exists(BIN), "stream_generate not built (run __graft_entry__.build())"
    r = subprocess.run([BIN, model, ",".join(map(str, prompt)), str(n), str(T), "1.2", "256", "0.1", str(seed),
                        str(prefill_mode)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    lines = r.stdout.split("\n")
    toks = [int(s.split()[1]) for s in lines if s.startswith("token ")]
    done = [s for s in lines if s.startswith("done ")]
    assert done and int(done[0].split()[1]) == len(toks) == n, r.stdout
    return toks


def test_host_loop_greedy_with_penalties(orc, tmp_path):
    m = tiny_lm(2030)
    model = str(tmp_path / "tiny.bin")
    _write_model(m, model)
    prompt = [1, 17, 333, 5, 4000]
    want, margins = _oracle_loop(orc, m, prompt, 40, 0.0, 7)
    assert min(margins) > 1e-3, "seeded model has a near-tie: pick another seed"
    assert _run(model, prompt, 40, 0.0, 7) == want


def test_host_loop_batched_prefill_greedy(orc, tmp_path):
    """The prompt through every layer at once (forward_batch,
    models/llm/qwen3_5.cpp:1164-1217: batched projections; here the cores
    take the whole prompt too -- anelm_full_attn_prefill over the fp16 ring,
    anelm_deltanet_prefill_from_proj over the conv ring and state), then the
    decode loop from the state it left: the same tokens as the oracle's
    single-token prefill and decode."""
    m = tiny_lm(2030)
    model = str(tmp_path / "tiny.bin")
    _write_model(m, model)
    prompt = [1, 17, 333, 5, 4000, 12, 77, 4095, 600, 31, 2, 999]
    want, margins = _oracle_loop(orc, m, prompt, 40, 0.0, 7)
    assert min(margins) > 1e-3, "seeded model has a near-tie: pick another seed"
    assert _run(model, prompt, 40, 0.0, 7, prefill_mode=1) == want


def test_host_loop_sampled(orc, tmp_path):
    """T 0.6 with the seeded draws: identical tokens up to the first draw that
    lands within 2e-5 of a CDF step (logits that agree to ~1e-6 cannot move a
    crossing farther away than that; after it the loops may part)."""
    m = tiny_lm(2031)
    model = str(tmp_path / "tiny.bin")
    _write_model(m, model)
    prompt = [3, 99, 2048]
    want, margins = _oracle_loop(orc, m, prompt, 24, 0.6, 15)
    k = next((i for i, g in enumerate(margins) if g < 2e-5), len(margins))
    assert k >= 8, "an early undecided draw: pick another seed"
    got = _run(model, prompt, 24, 0.6, 15)
    assert got[:k + 1] == want[:k + 1] or got[:k] == want[:k]
    assert all(0 <= t < m["dims"]["vocab"] for t in got)
