"""GPU parity of device-side token sampling (anelm_sample_token) against the
oracle's restatement of core/sampling.cpp:11-66 with the same uniform draw:
penalties over the recent-token window, greedy first maximum, temperature
softmax and the CDF draw, at the 4B vocabulary (248320 logits)."""
import numpy as np
import pytest
import torch

from gpu_util import to_dev, to_host

pytestmark = pytest.mark.gpu

VOCAB = 248320


def _case(seed, V=VOCAB, n_recent=300, scale=2.0):
    rng = np.random.default_rng(seed)
    logits = (scale * rng.standard_normal(V)).astype(np.float32)
    recent = rng.integers(0, V, n_recent).astype(np.int32)
    recent[::7] = recent[0]            # repeated tokens: one penalty, frequency x count
    return rng, logits, recent


def test_sample_greedy_with_penalties(anelm, orc, dev):
    rng, logits, recent = _case(900)
    # put the maximum on a recent token so the penalty decides the winner
    top = int(np.argmax(logits))
    recent[-1] = top
    lg, rc = to_dev(logits, dev), to_dev(recent, dev)
    for ctx, rep, freq in ((256, 1.2, 0.1), (16, 1.5, 0.0), (256, 1.0, 0.5), (0, 1.2, 0.1)):
        got = int(to_host(anelm.ops.sample_token(lg, rc, 0.0, rep, ctx, freq))[0])
        want, _ = orc.sample_token(logits, recent, 0.0, rep, ctx, freq, 0.5)
        assert got == want, (ctx, rep, freq)
    # no recent tokens, and first-of-equal maxima
    flat = np.zeros(VOCAB, np.float32)
    flat[[5000, 77, 123456]] = 3.0
    assert int(to_host(anelm.ops.sample_token(to_dev(flat, dev), None, 0.0))[0]) == 77


def test_sample_greedy_nan_layouts(anelm, orc, dev):
    """sampling.cpp:47-53 starts at max_i = 0 and moves on a strict >: a NaN
    at index 0 is never replaced (token 0), a NaN elsewhere never wins."""
    rng = np.random.default_rng(901)
    base = rng.standard_normal(VOCAB).astype(np.float32)
    top = int(np.argmax(base))
    cases = []
    a = base.copy(); a[0] = np.nan; cases.append(("nan at 0", a))
    a = base.copy(); a[top - 1] = np.nan; a[VOCAB - 1] = np.nan; cases.append(("nan elsewhere", a))
    a = np.full(VOCAB, -np.inf, np.float32); cases.append(("all -inf", a))
    a = np.full(VOCAB, np.nan, np.float32); cases.append(("all nan", a))
    a = base.copy(); a[0] = -np.inf; a[1:1000] = np.nan; cases.append(("-inf at 0, nan run", a))
    for name, lg in cases:
        want, _ = orc.sample_token(lg, np.zeros(0, np.int32), 0.0, 1.0, 0, 0.0, 0.5)
        got = int(to_host(anelm.ops.sample_token(to_dev(lg, dev), None, 0.0))[0])
        assert got == want, (name, got, want)
    assert orc.sample_token(cases[0][1], np.zeros(0, np.int32), 0.0, 1.0, 0, 0.0, 0.5)[0] == 0


def _exact_cdf(orc, logits, recent, T):
    """Float64 running sum of the exact softmax of the penalised logits times
    1/T (the fp32 values both implementations exponentiate)."""
    _, pen = orc.sample_token(logits, recent, 0.0, 1.2, 256, 0.1, 0.5)   # penalised logits
    z = (pen * (np.float32(1.0) / np.float32(T))).astype(np.float64)
    p = np.exp(z - z.max())
    return np.cumsum(p / p.sum())


def _gap(cum, tok, r):
    """Distance in cumulative probability between the draw r and token tok's
    interval (cum[tok-1], cum[tok]] of the exact distribution (0 inside)."""
    lo = cum[tok - 1] if tok > 0 else 0.0
    return max(0.0, lo - r, r - cum[tok])


@pytest.mark.parametrize("T", [0.6, 1.0, 1.7])
def test_sample_cdf_draw(anelm, orc, dev, T):
    """The drawn token.  Over 248320 terms the reference's sequential fp32
    sums -- the softmax normaliser and the running sum of the draw -- drift
    from the exact ones by up to ~4e-4 in cumulative probability at T 0.6 (a
    ~4e-6 term added to a sum near 0.5 rounds at 3e-8), which moves the
    crossing of many draws by tens of tokens.  The device sums per block in a
    tree and walks the crossing block with a wave scan, following the exact
    sums to ~1e-6.  So the device token's interval of the exact distribution
    lies within 2e-6 of r (and is the exact draw itself in most draws), while
    the oracle's lies within its own measured drift of r."""
    rng, logits, recent = _case(901 + int(10 * T))
    lg, rc = to_dev(logits, dev), to_dev(recent, dev)
    cum = _exact_cdf(orc, logits, recent, T)
    exact = 0
    for r in rng.uniform(0, 1, 40):
        want, adj = orc.sample_token(logits, recent, T, 1.2, 256, 0.1, float(r))
        rf = float(np.float32(r))                                  # the ABI takes r as a float
        cum32 = np.cumsum(adj.astype(np.float32), dtype=np.float32)   # sequential fp32 adds
        assert want == int(np.nonzero(cum32 >= rf)[0][0])           # the oracle's rule
        drift = float(np.max(np.abs(cum32 - cum)))
        assert _gap(cum, want, rf) <= drift + 1e-7
        got = int(to_host(anelm.ops.sample_token(lg, rc, T, 1.2, 256, 0.1, float(r)))[0])
        assert _gap(cum, got, rf) <= 2e-6, (T, r, got, want, _gap(cum, got, rf))
        exact += _gap(cum, got, rf) == 0.0
    assert exact >= 30, exact
    print(f"T={T}: 40 draws within 2e-6 of the exact CDF, {exact} on the exact token")
    # a draw above every running sum returns the last token
    assert int(to_host(anelm.ops.sample_token(lg, rc, T, 1.2, 256, 0.1, 2.0))[0]) == VOCAB - 1


def test_sample_peaked_distribution(anelm, orc, dev):
    """Low temperature over a few dominant logits: the draw picks among them
    as the exact distribution does, and as the oracle does (the mass sits on
    five terms, so the fp32 drift cannot move a crossing)."""
    rng, logits, recent = _case(902, scale=1.0)
    hot = rng.choice(VOCAB, 5, replace=False)
    logits[hot] += np.array([9.0, 8.5, 8.7, 9.2, 8.9], np.float32)
    lg, rc = to_dev(logits, dev), to_dev(recent, dev)
    cum = _exact_cdf(orc, logits, recent, 0.5)
    seen = set()
    for r in np.linspace(0.01, 0.99, 25):
        want, _ = orc.sample_token(logits, recent, 0.5, 1.2, 256, 0.1, float(r))
        got = int(to_host(anelm.ops.sample_token(lg, rc, 0.5, 1.2, 256, 0.1, float(r)))[0])
        assert _gap(cum, got, float(np.float32(r))) <= 2e-6, r
        if np.min(np.abs(cum - r)) > 1e-4:
            assert got == want, r
        seen.add(got)
    assert len(seen) >= 3
