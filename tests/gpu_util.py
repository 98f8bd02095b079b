"""Helpers for the GPU parity tests: host<->device copies and the parity bar.

The bar (fp16-input / fp32-accumulate outputs): rel-L2 <= 1e-3 and
max-abs <= 2e-2 against the oracle on the same seeded inputs.
"""
import numpy as np
import torch

REL_L2 = 1e-3
MAX_ABS = 2e-2


def to_dev(a, dev):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(dev).view(torch.float16)
    return torch.from_numpy(a).to(dev)


def to_host(t):
    torch.cuda.synchronize()
    if t.dtype == torch.float16:
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    return t.cpu().numpy()


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def assert_close(got, want, rel=REL_L2, max_abs=MAX_ABS, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what} shape {got.shape} != {want.shape}"
    assert np.all(np.isfinite(got)), f"{what} has non-finite values"
    r = rel_l2(got, want)
    m = float(np.max(np.abs(got - want))) if got.size else 0.0
    assert r <= rel and m <= max_abs, f"{what} rel-L2 {r:.3e} (<= {rel}), max-abs {m:.3e} (<= {max_abs})"
    return r, m
