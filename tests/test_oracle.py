"""Pins the CPU oracle (oracle/sampler_oracle.c) before it is trusted as the checker.

Every case either comes from the reference's own tests / fixtures
(tests/sample/sampler_test.cpp, reference/fixtures*/), or checks the oracle
against an independent formulation (numpy/scipy/torch, brute force, closed
forms) chosen so that a plausible slip (strict vs non-strict cutoff, wrong tie
order, dropped normalisation, off-by-one k) fails.
"""
import glob
import math
import os

import numpy as np
import pytest
from scipy.special import logsumexp

HERE = os.path.dirname(os.path.abspath(__file__))
F32, BF16, F16 = 0, 1, 2


def log(x):
    return np.log(np.asarray(x, np.float32)).astype(np.float32)


# ---------------------------------------------------------------------------
# Known answers ported from tests/sample/sampler_test.cpp
# ---------------------------------------------------------------------------

def test_greedy_returns_argmax(orc):  # sampler_test.cpp:41-44
    z = np.array([[1.0, 3.0, 2.0], [5.0, 0.0, -1.0]], np.float32)
    r = orc.sample(z)
    assert r["ids"].tolist() == [1, 0]


def test_temperature_zero_is_greedy(orc):  # :46-52
    z = np.array([[0.2, 0.9, 0.1, 0.4]], np.float32)
    r = orc.sample(z, T=[0.0], u=[0.7])
    assert r["ids"].tolist() == [orc.greedy_row(z[0])]


def test_top_k_keeps_exactly_k(orc):  # :54-61
    f = orc.filter_row([5.0, 1.0, 4.0, 2.0, 3.0], k=2)
    assert np.isfinite(f).sum() == 2
    assert np.isfinite(f[0]) and np.isfinite(f[2]) and not np.isfinite(f[1])


def test_top_p_smallest_prefix(orc):  # :63-74
    f = orc.filter_row(log([0.5, 0.3, 0.15, 0.05]), p=0.7)
    assert np.isfinite(f).tolist() == [True, True, False, False]


def test_top_p_is_strict_on_prior_mass(orc):
    # prior mass of the 3rd token is exactly 0.8 (in float64 of the float32 logs,
    # up to rounding); p just above keeps it, p at 0.79 does not.
    lg = log([0.5, 0.3, 0.15, 0.05])
    assert np.isfinite(orc.filter_row(lg, p=0.79)).sum() == 2
    assert np.isfinite(orc.filter_row(lg, p=0.81)).sum() == 3
    assert np.isfinite(orc.filter_row(lg, p=0.96)).sum() == 4


def test_min_p(orc):  # :76-87
    f = orc.filter_row(log([0.5, 0.3, 0.15, 0.05]), min_p=0.4)
    assert np.isfinite(f).tolist() == [True, True, False, False]


def test_same_uniforms_reproduce_different_diverge(orc):  # :126-134 (key -> uniforms)
    z = np.zeros((64, 16), np.float32)
    rng = np.random.default_rng(42)
    u1 = rng.random(64, dtype=np.float32)
    u2 = np.random.default_rng(7).random(64, dtype=np.float32)
    a1 = orc.sample(z, T=np.ones(64), u=u1)["ids"]
    a2 = orc.sample(z, T=np.ones(64), u=u1)["ids"]
    b = orc.sample(z, T=np.ones(64), u=u2)["ids"]
    assert (a1 == a2).all() and (a1 != b).any()
    # uniform row: inverse CDF picks floor(u * 16)
    assert (a1 == np.floor(u1.astype(np.float64) * 16).astype(int)).all()


def test_batched_shapes_and_logprob_nonpositive(orc):  # :136-142
    z = np.array([[1.0, 2.0, 3.0], [3.0, 2.0, 1.0]], np.float32)
    r = orc.sample(z, T=[1.0, 1.0], u=[0.3, 0.9], tlp=[0, 0])
    assert r["ids"].shape == (2,) and r["lp"].shape == (2,)
    assert (r["lp"] <= 0).all()


def test_top_logprobs_off_and_zero(orc):  # :144-161
    z = np.array([[1.0, 2.0, 3.0]], np.float32)
    r = orc.sample(z, T=[0.0], tlp=[-1], K_max=0)
    assert r["top_ids"].shape == (1, 0) and np.isnan(r["lp"][0])
    r = orc.sample(z, T=[0.0], tlp=[0], K_max=0)
    assert r["ids"].tolist() == [2] and r["lp"][0] <= 0


def test_top_logprobs_ranked(orc):  # :163-181
    z = np.array([[1.0, 4.0, 2.0, 3.0, 0.0]], np.float32)
    r = orc.sample(z, T=[0.0], tlp=[3], K_max=3)
    assert r["top_ids"][0].tolist() == [1, 3, 2]
    lp = r["top_lp"][0]
    assert lp[0] >= lp[1] >= lp[2] and (lp <= 0).all()
    assert r["ids"].tolist() == [1] and r["lp"][0] == pytest.approx(lp[0])


def test_full_top_k_is_normalised(orc):  # :183-192
    z = np.array([[0.5, 1.5, -0.5, 2.0]], np.float32)
    r = orc.sample(z, T=[0.0], tlp=[4], K_max=4)
    assert np.exp(r["top_lp"][0].astype(np.float64)).sum() == pytest.approx(1.0, abs=1e-6)


def test_top_logprobs_pre_temperature(orc):  # :194-203
    z = np.array([[1.0, 4.0, 2.0, 3.0]], np.float32)
    r = orc.sample(z, T=[0.8], tlp=[2], K_max=2, u=[0.5])
    assert r["top_ids"][0].tolist() == [1, 3]


# ---------------------------------------------------------------------------
# Real-logit known answers (reference/fixtures*/argmax.npy, fp16 logits)
# ---------------------------------------------------------------------------

FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "fixtures", "*")))


@pytest.mark.parametrize("fx", FIXTURES, ids=[os.path.basename(f) for f in FIXTURES])
def test_real_logit_greedy_fixture(orc, fx):
    logits = np.load(os.path.join(fx, "logits_last.npy"), allow_pickle=False)
    want = np.load(os.path.join(fx, "argmax.npy"), allow_pickle=False)
    assert logits.dtype == np.float16
    r = orc.sample(logits, T=np.zeros(1), tlp=[0])
    assert r["ids"].tolist() == want.tolist()
    z64 = logits.astype(np.float64)[0]
    assert r["lp"][0] == pytest.approx(z64[want[0]] - logsumexp(z64), abs=1e-6)


# ---------------------------------------------------------------------------
# Independent formulations
# ---------------------------------------------------------------------------

def test_lse_closed_form(orc):
    rng = np.random.default_rng(1)
    for scale in (0.1, 2.0, 30.0):
        z = (rng.standard_normal(5000) * scale).astype(np.float32)
        assert orc.lse_row(z) == pytest.approx(logsumexp(z.astype(np.float64)), abs=1e-9)
    # single finite entry among -inf: LSE equals it
    z = np.full(7, -np.inf, np.float32)
    z[3] = 1.25
    assert orc.lse_row(z) == 1.25


def test_top_k_against_sorted_threshold_with_ties(orc):
    rng = np.random.default_rng(2)
    for trial in range(200):
        V = int(rng.integers(1, 60))
        z = rng.integers(-4, 5, V).astype(np.float32)  # heavy ties
        k = int(rng.integers(1, V + 3))
        f = orc.filter_row(z, k=k)
        kk = min(k, V)
        tau = np.sort(z)[::-1][kk - 1]
        assert (np.isfinite(f) == (z >= tau)).all()
        assert np.isfinite(f).sum() >= kk


def _brute_top_p(zs, p):
    """Smallest n such that the first n entries of the (z desc, idx asc) order carry
    mass >= p; an independent statement of 'keep j iff prior mass < p'."""
    V = zs.size
    order = sorted(range(V), key=lambda i: (-zs[i], i))
    m = max(zs)
    w = [math.exp(float(zs[i]) - float(m)) if np.isfinite(zs[i]) else 0.0 for i in order]
    W = math.fsum(w)
    for n in range(1, V + 1):
        if math.fsum(w[:n]) >= p * W:
            return set(order[:n])
    return set(order)


def test_top_p_against_brute_force(orc):
    rng = np.random.default_rng(3)
    checked = 0
    for trial in range(400):
        V = int(rng.integers(1, 9))
        z = (rng.integers(-6, 7, V) * 0.5).astype(np.float32)  # ties included
        p = float(np.float32(rng.uniform(0.05, 0.999)))
        f = orc.filter_row(z, p=p)
        got = set(np.nonzero(np.isfinite(f))[0].tolist())
        # skip exact-boundary cases where float64 summation order could matter
        order = sorted(range(V), key=lambda i: (-z[i], i))
        w = np.exp(z[order].astype(np.float64) - z.max())
        cs = np.cumsum(w) / w.sum()
        if np.min(np.abs(cs - p)) < 1e-12:
            continue
        assert got == _brute_top_p(z, p), (z, p)
        checked += 1
    assert checked > 300


def test_draw_is_inverse_cdf(orc):
    z = np.array([0.0, 1.0, -1.0, 2.0, 0.5], np.float32)
    q = np.exp(z.astype(np.float64) - z.max())
    q /= q.sum()
    N = 20000
    counts = np.zeros(5, int)
    for j in range(N):
        i, _ = orc.draw_row(z, float(np.float32((j + 0.5) / N)))
        counts[i] += 1
    assert np.abs(counts - q * N).max() <= 2


def test_draw_ascending_vocab_order(orc):
    # equal weights: u in [j/4, (j+1)/4) picks the j-th kept entry in index order
    zs = np.array([-np.inf, 0.0, -np.inf, 0.0, 0.0, -np.inf, 0.0], np.float32)
    kept = [1, 3, 4, 6]
    for j in range(4):
        i, _ = orc.draw_row(zs, (j + 0.5) / 4)
        assert i == kept[j]


def test_bf16_rounding_matches_torch(orc):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(4)
    base = (rng.standard_normal(1000).astype(np.float32).view(np.uint32) & np.uint32(0xFFFF0000))
    halfway = (base | np.uint32(0x8000)).view(np.float32)  # exactly between two bf16 values
    x = np.concatenate([rng.standard_normal(2000).astype(np.float32) * 10, halfway])
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    got = np.array([orc.round_bf16(float(v)) for v in x], np.float32)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()
    for v in (0.7, 0.9, 0.95, 0.8, 1.2):  # values the configs use
        assert orc.round_bf16(v) == float(torch.tensor(v).to(torch.bfloat16))


def test_f16_rounding_matches_numpy(orc):
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(3000).astype(np.float32) * 100,
                        rng.standard_normal(1000).astype(np.float32) * 1e-6,  # subnormal halves
                        np.array([65504, 65519, 65520, 1e6, -7e-8, 3e-8], np.float32)])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).astype(np.float32)
    got = np.array([orc.round_f16(float(v)) for v in x], np.float32)
    assert np.array_equal(got, want)


def test_bf16_temperature_and_division(orc):
    # D1: z' = bf16(z / bf16(T)); T = 0.7 becomes 0.69921875
    bits = np.array([[0x4000, 0x3f80, 0xbf80]], np.uint16)  # 2, 1, -1
    out = orc.filter_row(np.array([2.0, 1.0, -1.0], np.float32), T=0.7, dtype=BF16)
    Tb = np.float32(0.69921875)
    want = [orc.round_bf16(float(np.float32(v) / Tb)) for v in (2.0, 1.0, -1.0)]
    assert out.tolist() == want
    assert bits.shape == (1, 3)


def test_nan_reads_as_neg_inf_and_degenerate_rows(orc):
    z = np.array([[np.nan, 1.0, np.nan, 1.0]], np.float32)
    assert orc.sample(z)["ids"].tolist() == [1]
    allneg = np.full((1, 5), -np.inf, np.float32)
    r = orc.sample(allneg, T=[1.0], u=[0.99], tlp=[0])
    # nothing to draw: index 0, the argmax MLX's Gumbel-max categorical takes
    assert r["ids"].tolist() == [0] and np.isnan(r["lp"][0])
    assert orc.sample(allneg)["ids"].tolist() == [0]
    inf = np.array([[1.0, np.inf, 3.0, np.inf]], np.float32)
    r = orc.sample(inf, T=[1.0], u=[0.75])
    assert r["ids"].tolist() == [3]  # mass split evenly between the two +inf entries


def test_parameter_sanitisation(orc):
    z = np.array([[0.0, 3.0, 1.0, 2.0]], np.float32)
    for T in (np.nan, np.inf, -1.0, 0.0):
        assert orc.sample(z, T=[T], u=[0.1])["ids"].tolist() == [1]
    # k > V clamps, k <= 0 and p outside (0, 1) disable
    a = orc.sample(z, T=[1.0], k=[100], u=[0.2])["ids"]
    b = orc.sample(z, T=[1.0], k=[0], p=[1.5], u=[0.2])["ids"]
    c = orc.sample(z, T=[1.0], p=[-0.2], u=[0.2])["ids"]
    assert a.tolist() == b.tolist() == c.tolist()


def test_ambiguity_flags(orc):
    # two tokens, probs (0.5, 0.5): the cutoff prior mass 0.5 sits exactly at p=0.5
    z = np.array([[0.0, 0.0, -30.0]], np.float32)
    r = orc.sample(z, T=[1.0], p=[0.5], u=[0.3])
    assert r["flags"][0] & orc.FLAG_TOPP_AMBIG
    r = orc.sample(z, T=[1.0], p=[0.7], u=[0.3])
    assert not (r["flags"][0] & orc.FLAG_TOPP_AMBIG)
    # draw boundary: u at the cumulative mass of the first kept token
    r = orc.sample(z, T=[1.0], u=[0.5])
    assert r["flags"][0] & orc.FLAG_DRAW_AMBIG


def test_min_p_one_keeps_the_max_and_is_not_ambiguous(orc):
    """min_p = 1 keeps exactly the row max (and its ties); the max's own
    weight is 1, so it gives no ambiguity margin."""
    z = np.array([[0.5, 2.0, 1.0, 2.0, -1.0], [0.5, 3.0, 1.0, 2.0, -1.0]], np.float32)
    for u in (0.0, 0.3, 0.6, 0.99):
        r = orc.sample(z, T=[1.0, 1.0], min_p=[1.0, 1.0], u=[u, u])
        assert r["ids"][0] in (1, 3) and r["ids"][1] == 1
        assert not (r["flags"] & orc.FLAG_MINP_AMBIG).any()
    r = orc.sample(z[:1], T=[1.0], min_p=[1.0], u=[0.3])
    assert r["ids"].tolist() == [1]
    r = orc.sample(z[:1], T=[1.0], min_p=[1.0], u=[0.6])
    assert r["ids"].tolist() == [3]


def test_admissible_ids(orc):
    """The checker of ambiguous rows: the ids a row can produce when p, u and
    min_p move by up to 1e-6."""
    z = np.array([0.0, 0.0, -30.0], np.float32)
    # top-p cutoff exactly at p = 0.5: {0} or {0, 1} kept
    assert orc.admissible(z, orc.F32, T=1.0, p=0.5, u=0.3) == [0]
    assert orc.admissible(z, orc.F32, T=1.0, p=0.5, u=0.7) == [0, 1]
    # draw boundary at u = 0.5: either side
    assert orc.admissible(z, orc.F32, T=1.0, u=0.5) == [0, 1]
    # an unambiguous row admits only the oracle's id
    assert orc.admissible(z, orc.F32, T=1.0, u=0.25) == [0]
    assert orc.admissible(z, orc.F32, T=0.0) == [0]
    # min_p at a kept weight: e^-1 at min_p = e^-1 (rounded to fp32)
    zz = np.array([1.0, 0.0, -5.0], np.float32)
    mp = float(np.float32(np.exp(-1.0)))
    a = orc.admissible(zz, orc.F32, T=1.0, min_p=mp, u=0.9)
    assert a == [0, 1], a
    # nothing to draw: index 0
    assert orc.admissible(np.full(4, -np.inf, np.float32), orc.F32, T=1.0, u=0.7) == [0]


def test_admissible_covers_perturbed_oracle(orc):
    """Brute force: the oracle's own ids with p, u and min_p moved anywhere in
    [-1e-6, 1e-6] all lie in the admissible set, and a row the oracle does not
    flag admits only its id."""
    rng = np.random.default_rng(404)
    eps = 1e-6
    for trial in range(40):
        V = int(rng.integers(2, 40))
        z = rng.integers(-4, 5, V).astype(np.float32) * np.float32(0.5)  # ties and round masses
        T = float(rng.choice([0.5, 1.0]))
        k = int(rng.choice([0, 0, 3]))
        p = float(rng.choice([1.0, 0.5, 0.75, 0.9]))
        mp = float(rng.choice([0.0, 0.0, 0.25, 1.0]))
        u = float(rng.choice([0.0, 0.25, 0.5, 0.75, float(rng.random())]))
        a = orc.admissible(z, orc.F32, T=T, k=k, p=p, min_p=mp, u=u)
        assert a is not None
        base = orc.sample(z[None], T=[T], k=[k], p=[p], min_p=[mp], u=[u])
        assert base["ids"][0] in a
        if not (base["flags"][0] & orc.AMBIG):
            assert a == [int(base["ids"][0])], (trial, a, base)
        for d in np.linspace(-eps, eps, 9):
            for which in ("p", "u", "mp"):
                pp = p + d if which == "p" and p < 1.0 else p
                uu = min(max(u + d, 0.0), 0.9999999) if which == "u" else u
                mm = mp * (1 + d) if which == "mp" and mp > 0 else mp
                mm = min(mm, 1.0)
                r = orc.sample(z[None], T=[T], k=[k], p=[np.float32(pp)], min_p=[np.float32(mm)],
                               u=[np.float32(uu)])
                assert r["ids"][0] in a, (trial, which, d, r["ids"][0], a)


def test_workloads_are_deterministic(orc):
    from mlxforge_amd import workloads
    a, b = workloads.make(1), workloads.make(1)
    assert np.array_equal(a.logits, b.logits) and a.B == 1 and a.V == 128256
    assert a.algorithmic_bytes() == 513048
    assert workloads.make(3).algorithmic_bytes() == 19448576


def test_min_p_in_the_batched_oracle(orc):
    """The batched oracle's min_p (after top-p) equals filtering the row with
    the filter stage and drawing from what is left, and keeps exactly the
    weights exp(z' - max z') >= min_p (brute force)."""
    rng = np.random.default_rng(31)
    B, V = 24, 300
    z = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    T = rng.uniform(0.5, 1.5, B).astype(np.float32)
    k = rng.choice([0, 5, 40], B).astype(np.int32)
    p = rng.choice([1.0, 0.9, 0.6], B).astype(np.float32)
    mp = rng.choice([0.0, 0.01, 0.1, 0.5, 1.0], B).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    r = orc.sample(z, T=T, k=k, p=p, min_p=mp, u=u, tlp=np.full(B, -1, np.int32))
    for i in range(B):
        f = orc.filter_row(z[i], T=float(T[i]), k=int(k[i]), p=float(p[i]), min_p=float(mp[i]))
        # brute force of the min_p step alone on the top-k / top-p survivors
        g = orc.filter_row(z[i], T=float(T[i]), k=int(k[i]), p=float(p[i]))
        fin = np.isfinite(g)
        w = np.exp(g[fin].astype(np.float64) - g[fin].max())
        keep = np.zeros(V, bool)
        keep[np.nonzero(fin)[0]] = w >= float(mp[i]) if mp[i] > 0 else True
        assert np.array_equal(np.isfinite(f), keep), i
        if not (r["flags"][i] & (orc.FLAG_DRAW_AMBIG | orc.FLAG_MINP_AMBIG | orc.FLAG_TOPP_AMBIG)):
            assert r["ids"][i] == orc.draw_row(f, float(u[i]))[0], i


def test_repetition_penalty(orc):  # tests/sample/sampler_test.cpp:89-98
    f = orc.apply_penalties([2.0, 1.0, 0.5], [0], rep=4.0)
    assert f.tolist() == [0.5, 1.0, 0.5]
    # a negative seen logit is multiplied (pushed further down)
    assert orc.apply_penalties([-2.0, 1.0], [0], rep=4.0).tolist() == [-8.0, 1.0]


def test_frequency_and_presence_penalties(orc):  # :100-115
    hist = [1, 1, 2]
    assert orc.apply_penalties([0.0] * 4, hist, freq=0.5).tolist() == [0.0, -1.0, -0.5, 0.0]
    assert np.allclose(orc.apply_penalties([0.0] * 4, hist, pres=0.7), [0.0, -0.7, -0.7, 0.0])


def test_repetition_penalty_moves_greedy(orc):  # :117-124
    f = orc.apply_penalties([2.0, 1.0, 0.5], [0], rep=4.0)
    assert orc.greedy_row(f) == 1


def test_penalty_sanitisation_and_rounding(orc):
    # off: rep 1 / non-finite / non-positive, freq and pres 0 / non-finite
    for kw in (dict(rep=1.0), dict(rep=float("nan")), dict(rep=-2.0), dict(freq=float("inf")),
               dict(pres=float("nan"))):
        assert orc.apply_penalties([2.0, 1.0], [0, 1], **kw).tolist() == [2.0, 1.0]
    # ids outside [0, V) are ignored
    assert orc.apply_penalties([2.0, 1.0], [-1, 7], rep=2.0).tolist() == [2.0, 1.0]
    # bf16: every step rounds to bf16 (0.3 -> 0.30078125, 1/3 of 1 -> 0.333984375)
    b = orc.apply_penalties([1.0, 0.0], [0, 0, 0], rep=3.0, freq=0.3, dtype=orc.BF16)
    x = orc.round_bf16(1.0 / orc.round_bf16(3.0))
    x = orc.round_bf16(x - orc.round_bf16(3.0 * orc.round_bf16(0.3)))
    assert b[0] == x and b[1] == 0.0
    # against a float64 restatement with rounding after every op (fp32 rows)
    rng = np.random.default_rng(4)
    z = (rng.standard_normal(50) * 3).astype(np.float32)
    h = rng.integers(0, 50, 80)
    got = orc.apply_penalties(z, h, rep=1.7, freq=0.25, pres=0.4)
    exp = z.copy()
    for i, c in zip(*np.unique(h, return_counts=True)):
        x = np.float32(z[i])
        x = np.float32(x / np.float32(1.7)) if x > 0 else np.float32(x * np.float32(1.7))
        x = np.float32(x - np.float32(np.float32(c) * np.float32(0.25)))
        exp[i] = np.float32(x - np.float32(0.4))
    assert np.array_equal(got, exp)


def test_philox_known_answers(orc):
    """Philox4x32-10 against the published known-answer vectors of its authors'
    Random123 library (counter, key -> output)."""
    assert orc.philox4x32_10([0, 0, 0, 0], [0, 0]) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    f = 0xFFFFFFFF
    assert orc.philox4x32_10([f, f, f, f], [f, f]) == [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert orc.philox4x32_10([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344],
                             [0xA4093822, 0x299F31D0]) == [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]


def test_uniforms_are_a_function_of_seed_and_step(orc):
    seeds = np.array([0, 1, 2**63 + 5, 42], np.uint64)
    a = orc.uniforms(seeds, 7)
    assert np.array_equal(a, orc.uniforms(seeds, 7))          # same seed, same step: replay
    assert not np.array_equal(a, orc.uniforms(seeds, 8))      # next step draws anew
    assert ((a >= 0) & (a < 1)).all()
    # u is the top 24 bits of the first output word
    w = orc.philox4x32_10([7, 0, 0, 0], [42, 0])[0]
    assert a[3] == np.float32((w >> 8) * 2.0 ** -24)
    # roughly uniform over many steps
    u = orc.uniforms(np.full(20000, 9, np.uint64), np.arange(20000, dtype=np.uint64))
    assert abs(float(u.mean()) - 0.5) < 0.01 and abs(float((u < 0.1).mean()) - 0.1) < 0.01


def test_grammar_mask(orc):
    """row + fp32 mask (src/runtime/worker.cpp:142-179,455-459): allowed
    entries keep their value, the rest are -inf; an all-disallowed row is left
    as is; bits pack little-endian within each word."""
    z = np.array([1.5, -2.0, 0.25, 7.0], np.float32)
    m = orc.apply_mask(z, [True, False, True, False])
    assert m.tolist() == [1.5, -np.inf, 0.25, -np.inf]
    assert orc.apply_mask(z, [False] * 4).tolist() == z.tolist()
    # token 33 is bit 1 of word 1
    assert orc.pack_bits([[True, False, True] + [False] * 30 + [True]]).tolist() == [[0b101, 0b10]]
    assert orc.greedy_row(orc.apply_mask(z, [True, False, True, False])) == 0
