"""GPU parity of the row-histogram path (bf16 logits, no top_logprobs, V >=
32768): every row kind against the CPU oracle, and bit for bit against the
per-slice path on the same inputs (a call with K_max > 0 takes the per-slice
path; both compute the same integer masses, so the ids agree exactly).

Covers the rows the histogram bins decide themselves and the rows they hand to
the fallback kernel (NaN, +-inf, logits >= 256 in magnitude, rows of zeros or
of values within 2^-28 of zero, cutoffs next to those bins).
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - collected on CPU-only hosts too
    pytest.skip("no GPU", allow_module_level=True)

from mlxforge_amd import workloads  # noqa: E402
from tests import gpu_util as gu  # noqa: E402


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _bits(z):
    return workloads.to_bf16_bits(np.nan_to_num(z, nan=0.0, posinf=3e38, neginf=-3e38))


def _params(rng, B, kinds=None):
    """Per-row parameters over every row kind."""
    T = np.zeros(B, np.float32)
    k = np.zeros(B, np.int32)
    p = np.ones(B, np.float32)
    mp = np.zeros(B, np.float32)
    kinds = kinds or ["greedy", "temp", "klist", "khist", "topp", "k_topp", "minp", "all"]
    for r in range(B):
        kind = kinds[r % len(kinds)]
        if kind != "greedy":
            T[r] = rng.uniform(0.4, 1.5)
        if kind in ("klist", "k_topp", "all"):
            k[r] = rng.integers(1, 64)
        if kind == "khist":
            k[r] = rng.choice([64, 100, 1000, 5000, 40000])
        if kind in ("topp", "k_topp", "all"):
            p[r] = rng.choice([0.3, 0.8, 0.9, 0.95, 0.999])
        if kind in ("minp", "all"):
            mp[r] = rng.choice([0.001, 0.05, 0.3, 1.0])
    tlp = rng.integers(-1, 1, B).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    return T, k, p, mp, tlp, u


def _check(host, T, k, p, mp, tlp, u, label, V=None, dev=None):
    dev = gu.to_device(host, "bf16") if dev is None else dev
    say(f"[rowhist] {label}")
    g = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u, min_p=mp, V=V)
    o = gu.oracle_sample(host, "bf16", T=T, k=k, p=p, tlp=tlp, u=u, min_p=mp, V=V)
    rep = gu.compare(g, o, "bf16", tlp=tlp, label=label)
    # the per-slice path (K_max > 0) on the same inputs: the same ids
    s = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u, min_p=mp, V=V, K_max=1)
    assert np.array_equal(g["ids"], s["ids"]), (label, np.nonzero(g["ids"] != s["ids"])[0][:8])
    # determinism
    g2 = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u, min_p=mp, V=V)
    assert np.array_equal(g["ids"], g2["ids"])
    assert np.array_equal(g["lp"].view(np.uint32), g2["lp"].view(np.uint32))
    return rep


@pytest.mark.parametrize("V,B", [(32768, 16), (32769, 16), (50001, 16), (151936, 16), (262144, 16),
                                 (40000, 1), (65536 + 8192 * 3 + 5, 9), (151936, 80), (32768, 72),
                                 (32769, 72), (65536 + 8192 * 3 + 5, 70), (262144, 72), (458752, 65),
                                 (458752 + 8, 65)])
def test_row_kinds(V, B):
    """B <= 64: split call (the chunks counted by their own workgroups, XCD
    groups of 8 rows, a partial last group for B = 1 and 9); B > 64: one
    workgroup per row, 16-bit counters for the halves of each chunk (the walk
    picks one of eight), up to V = 458752 (the largest whose half chunks hold
    at most 65535 logits; one more takes the per-slice path)."""
    rng = np.random.default_rng(900 + V % 97 + B)
    z = np.empty((B, V), np.float32)
    for r in range(B):
        shape = r % 4
        if shape == 0:
            z[r] = rng.standard_normal(V) * 3
            z[r, rng.integers(0, V)] = 15.0
        elif shape == 1:
            z[r] = rng.standard_normal(V) * 0.1
        elif shape == 2:
            z[r] = rng.gumbel(size=V) * 2.5 - 1.1 * np.log(np.arange(1, V + 1))
        else:
            z[r] = rng.standard_normal(V) * 1.5
    T, k, p, mp, tlp, u = _params(rng, B)
    _check(_bits(z), T, k, p, mp, tlp, u, f"row kinds V={V}")


@pytest.mark.parametrize("B", [16, 72])
def test_heavy_ties_and_flat_rows(B):
    """Few distinct values: every cutoff lands in a tie group spread over the
    four chunks (B = 16) or the eight half chunks (B = 72)."""
    rng = np.random.default_rng(31 + B)
    V = 120000
    z = np.empty((B, V), np.float32)
    for r in range(B):
        if r % 3 == 0:
            z[r] = rng.integers(-3, 4, V).astype(np.float32)
        elif r % 3 == 1:
            z[r] = np.round(rng.standard_normal(V) * 0.1, 2)
        else:
            z[r] = rng.integers(0, 2, V).astype(np.float32) * 0.5
    T, k, p, mp, tlp, u = _params(rng, B)
    for uu in (u, np.full(B, 0.0, np.float32), np.full(B, 0.999999, np.float32)):
        _check(_bits(z), T, k, p, mp, tlp, uu, f"heavy ties B={B}")


@pytest.mark.parametrize("reps", [1, 6])
def test_fallback_rows(reps):
    """Rows the bins cannot decide: the per-slice fallback in the same
    workgroup finishes them.  reps=1 (12 rows) takes the split call (chunk
    workgroups, then one deciding workgroup per row), reps=6 (72 rows) the
    one-workgroup-per-row call."""
    rng = np.random.default_rng(77)
    B, V = 12, 40000
    z = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    bits = _bits(z)
    bits[0, 123] = 0x7FC0                       # a positive NaN (reads as -inf)
    bits[1, 5] = 0x7F80                         # +inf
    bits[2, 999] = _bits(np.array([300.0], np.float32))[0]  # a logit >= 256
    bits[3, :] = 0                              # all zeros
    bits[4, :] = 0xFF80                         # all -inf
    bits[5, :] = _bits((rng.standard_normal(V) * 1e-10).astype(np.float32))  # all tiny
    bits[6, :] = _bits((rng.standard_normal(V) * 2 - 300).astype(np.float32))  # all below -256
    bits[7, ::3] = 0xFFC0                       # negative NaNs
    bits[8, ::2] = 0                            # half zeros: cutoffs near the tiny bin
    bits[9, ::5] = _bits(np.array([-400.0], np.float32))[0]
    bits[10, 7] = 0xFF80                        # one -inf
    T = np.array([1.0, 1.0, 0.8, 1.0, 1.0, 1.0, 1.0, 0.9, 1.0, 1.2, 0.7, 0.0], np.float32)
    k = np.array([0, 0, 10, 0, 0, 0, 100, 0, 30000, 0, 0, 0], np.int32)
    p = np.array([0.9, 1.0, 1.0, 0.5, 1.0, 0.9, 1.0, 0.95, 0.9, 0.8, 1.0, 1.0], np.float32)
    mp = np.array([0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.1, 0.0, 0.0, 0.5, 0.0], np.float32)
    tlp = np.zeros(B, np.int32)
    u = rng.random(B).astype(np.float32)
    if reps > 1:
        bits, T, k, p, mp, tlp = (np.concatenate([v] * reps) for v in (bits, T, k, p, mp, tlp))
        u = rng.random(B * reps).astype(np.float32)
    _check(np.ascontiguousarray(bits), T, k, p, mp, tlp, u, f"fallback rows x{reps}")


def test_padded_rows_and_benchmark_configs():
    """row_stride > V (bucket padding) and the two bf16 benchmark configs."""
    rng = np.random.default_rng(5)
    B, V = 6, 65536 + 24
    full = _bits((rng.standard_normal((B, V + 40)) * 3).astype(np.float32))
    dev = gu.to_device(full, "bf16")[:, :V]
    T, k, p, mp, tlp, u = _params(rng, B)
    _check(np.ascontiguousarray(full[:, :V]), T, k, p, mp, tlp, u, "padded", dev=dev)
    for cfg in (2, 5):
        wl = workloads.make(cfg)
        rep = _check(wl.logits, wl.T, wl.k, wl.p, np.zeros(wl.B, np.float32), wl.tlp, wl.u, f"C{cfg}")
        say(f"[rowhist] C{cfg}: {rep}")
