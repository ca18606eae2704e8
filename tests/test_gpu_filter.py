"""GPU parity of the filter helpers (Sampler::apply_top_k / apply_top_p /
apply_min_p, src/sample/sampler.h:63-69, src/sample/sampler.cpp:63-93) and of
their composition after the temperature division (mlxf_filter_logits,
sampler.cpp:158-163): the reference's own filter cases
(tests/sample/sampler_test.cpp:54-87), then random rows of every dtype bit for
bit against the oracle's filter stage (orc_filter_row), in place and with
padded rows, ties and non-finite logits.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - collected on CPU-only hosts too
    pytest.skip("no GPU", allow_module_level=True)

from mlxforge_amd import sampler, workloads  # noqa: E402
from oracle import oracle as orc  # noqa: E402
from tests import gpu_util as gu  # noqa: E402

CODES = {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}


def say(msg):
    print(msg, flush=True)


def _host(z, dtype):
    if dtype == "f32":
        return z.astype(np.float32)
    if dtype == "bf16":
        return workloads.to_bf16_bits(z)
    return z.astype(np.float16)


def _vals(host, dtype):
    """float32 values of the host array (NaN kept)."""
    if dtype == "bf16":
        return workloads.bf16_bits_to_f32(host)
    return host.astype(np.float32)


def _out_vals(t, dtype):
    a = t.cpu()
    if dtype == "bf16":
        return workloads.bf16_bits_to_f32(a.view(torch.int16).numpy().view(np.uint16))
    return a.float().numpy()


def _same(a, b):
    """Bit-equal as float32 (so -0 and +0 differ, and -inf positions must agree)."""
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _compare(got, vals, dtype, label, per_row=None, **kw):
    """Each row bit for bit against the oracle's filter stage, except rows whose
    top-p or min_p cutoff the oracle flags as ambiguous (within 1e-6 of the
    compared quantity: the exclusion rule) and that differ: those are counted,
    at most a quarter of the rows, and must agree wherever both keep an
    entry."""
    B = got.shape[0]
    excluded = 0
    for r in range(B):
        args = dict(kw)
        if per_row:
            args.update({key: v[r] for key, v in per_row.items()})
        exp, flags = orc.filter_row(vals[r], dtype=CODES[dtype], with_flags=True, **args)
        if flags and not _same(got[r], exp):
            excluded += 1
            both = np.isfinite(got[r]) & np.isfinite(exp)
            assert _same(got[r][both], exp[both]), (label, r)
        else:
            assert _same(got[r], exp), (label, r, np.nonzero(got[r].view(np.uint32) != exp.view(np.uint32))[0][:5])
    assert excluded * 4 <= B, (label, excluded)
    return excluded


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_reference_filter_cases(dtype):
    """tests/sample/sampler_test.cpp:54-87."""
    say(f"[filter] reference cases {dtype}")
    lg = np.log(np.array([0.5, 0.3, 0.15, 0.05], np.float32))
    dev = gu.to_device(_host(np.array([[5.0, 1.0, 4.0, 2.0, 3.0]], np.float32), dtype), dtype)
    f = _out_vals(sampler.apply_top_k(dev, 2), dtype)[0]
    assert np.isfinite(f).sum() == 2 and np.isfinite(f[0]) and np.isfinite(f[2]) and not np.isfinite(f[1])
    dev = gu.to_device(_host(lg[None, :], dtype), dtype)
    f = _out_vals(sampler.apply_top_p(dev, 0.7), dtype)[0]
    assert np.isfinite(f).tolist() == [True, True, False, False]
    f = _out_vals(sampler.apply_min_p(dev, 0.4), dtype)[0]
    assert np.isfinite(f).tolist() == [True, True, False, False]
    # kept entries keep their value
    assert f[0] == _vals(_host(lg, dtype), dtype)[0]


def _rows(rng, B, V, dtype):
    z = np.empty((B, V), np.float32)
    for r in range(B):
        kind = r % 4
        if kind == 0:
            z[r] = rng.standard_normal(V) * 3
        elif kind == 1:
            z[r] = rng.gumbel(size=V) * 2.5 - 1.1 * np.log(np.arange(1, V + 1))
        elif kind == 2:
            z[r] = np.round(rng.standard_normal(V) * 2, 1)  # many exact ties
        else:
            z[r] = rng.standard_normal(V) * 0.3
            z[r, rng.integers(0, V)] = 12.0
    return z


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("V", [7, 1000, 40000, 151936])
def test_helpers_match_oracle(dtype, V):
    rng = np.random.default_rng(4000 + V + len(dtype))
    B = 8
    host = _host(_rows(rng, B, V, dtype), dtype)
    vals = _vals(host, dtype)
    dev = gu.to_device(host, dtype)
    code = CODES[dtype]
    for k in (1, 3, 50, V // 2, V, V + 5):
        say(f"[filter] top-k {dtype} V={V} k={k}")
        got = _out_vals(sampler.apply_top_k(dev, k), dtype)
        exp = np.stack([orc.filter_row(vals[r], k=k, dtype=code) for r in range(B)])
        assert _same(got, exp), k  # comparisons only: never ambiguous
    for p in (0.05, 0.5, 0.9, 0.999):
        say(f"[filter] top-p {dtype} V={V} p={p}")
        _compare(_out_vals(sampler.apply_top_p(dev, p), dtype), vals, dtype, f"p={p}", p=p)
    for mp in (0.001, 0.1, 0.5, 1.0):
        say(f"[filter] min-p {dtype} V={V} min_p={mp}")
        _compare(_out_vals(sampler.apply_min_p(dev, mp), dtype), vals, dtype, f"min_p={mp}", min_p=mp)
    # off values keep every entry
    for call, arg in ((sampler.apply_top_k, 0), (sampler.apply_top_p, 1.0), (sampler.apply_min_p, 0.0)):
        assert _same(_out_vals(call(dev, arg), dtype), vals)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_filter_logits_per_row(dtype):
    """Temperature, then top-k, top-p, min_p, per row, as the sampling call."""
    rng = np.random.default_rng(77 + len(dtype))
    B, V = 24, 50001
    host = _host(_rows(rng, B, V, dtype), dtype)
    vals = _vals(host, dtype)
    T = rng.uniform(0.3, 1.5, B).astype(np.float32)
    T[::7] = 0.0  # no division
    k = rng.choice([0, 1, 5, 64, 1000, 60000], B).astype(np.int32)
    p = rng.choice([1.0, 0.3, 0.8, 0.95], B).astype(np.float32)
    mp = rng.choice([0.0, 0.01, 0.2], B).astype(np.float32)
    say(f"[filter] filter_logits {dtype}")
    d = lambda a, t: torch.as_tensor(a, dtype=t).cuda()
    got = _out_vals(sampler.filter_logits(gu.to_device(host, dtype), temperature=d(T, torch.float32),
                                          top_k=d(k, torch.int32), top_p=d(p, torch.float32),
                                          min_p=d(mp, torch.float32)), dtype)
    n = _compare(got, vals, dtype, "per row", per_row={"T": [float(x) for x in T], "k": [int(x) for x in k],
                                                      "p": [float(x) for x in p], "min_p": [float(x) for x in mp]})
    say(f"[filter] per row: {n} of {B} rows ambiguous")


def test_in_place_padded_and_non_finite():
    rng = np.random.default_rng(5)
    B, V, pad = 6, 3000, 40
    z = (rng.standard_normal((B, V + pad)) * 2).astype(np.float32)
    z[0, 17] = np.nan
    z[1, :] = -np.inf
    z[2, 5] = np.inf
    z[2, 9] = np.inf
    z[3, ::2] = -0.0
    z[3, 1::2] = 0.0
    z[4, 100] = -np.inf
    full = torch.from_numpy(z).cuda()
    view = full[:, :V]
    vals = np.where(np.isnan(z[:, :V]), -np.inf, z[:, :V]).astype(np.float32)
    for p in (0.5, 0.9):
        say(f"[filter] padded p={p}")
        _compare(sampler.apply_top_p(view, p).cpu().numpy(), vals, "f32", f"padded p={p}", p=p)
    say("[filter] in place")
    exp = np.stack([orc.filter_row(vals[r], k=10) for r in range(B)])
    out = sampler.apply_top_k(view, 10, out=view)
    assert out.data_ptr() == view.data_ptr()
    assert _same(view.cpu().numpy(), exp)
    # the padding is untouched
    assert _same(full[:, V:].cpu().numpy(), z[:, V:])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("off", [0, 3])
def test_in_place_several_workgroups_per_row(dtype, off):
    """Rows split over several workgroups (G > 1), filtered in place, with the
    view's base 16-byte aligned (off = 0: 16-byte loads and stores) or not
    (off = 3: element loads and stores); the columns around the view keep
    their values."""
    rng = np.random.default_rng(900 + off + len(dtype))
    B, V, pad = 8, 40000, 24
    z = _rows(rng, B, V + pad, dtype)
    host = _host(z, dtype)
    full = gu.to_device(host, dtype)
    view = full[:, off:off + V]
    vals = _vals(host, dtype)[:, off:off + V]
    T = rng.uniform(0.5, 1.2, B).astype(np.float32)
    k = np.array([0, 40, 0, 5000, 0, 1, 0, 20000], np.int32)
    p = np.array([0.9, 1.0, 0.5, 0.95, 0.3, 1.0, 0.99, 0.8], np.float32)
    mp = np.array([0.0, 0.0, 0.02, 0.0, 0.0, 0.0, 0.001, 0.1], np.float32)
    say(f"[filter] in place, G > 1, {dtype} off={off}")
    d = lambda a, t: torch.as_tensor(a, dtype=t).cuda()
    before = _out_vals(full, dtype)
    out = sampler.filter_logits(view, temperature=d(T, torch.float32), top_k=d(k, torch.int32),
                                top_p=d(p, torch.float32), min_p=d(mp, torch.float32), out=view)
    assert out.data_ptr() == view.data_ptr()
    after = _out_vals(full, dtype)
    _compare(after[:, off:off + V], vals, dtype, f"in place off={off}",
             per_row={"T": [float(x) for x in T], "k": [int(x) for x in k], "p": [float(x) for x in p],
                      "min_p": [float(x) for x in mp]})
    assert _same(after[:, :off], before[:, :off]) and _same(after[:, off + V:], before[:, off + V:])


def test_overlap_refused():
    x = torch.zeros((4, 100), dtype=torch.float32, device="cuda")
    with pytest.raises(Exception):
        sampler.apply_top_k(x[:, :90], 3, out=x[:, 5:95])
