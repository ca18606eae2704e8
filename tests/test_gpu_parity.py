"""GPU parity: the HIP sampler (through the C ABI) against the CPU oracle.

Covers the five benchmark configurations at full size, the reference's own
known answers and real-logit fixtures, and the edge cases the reference's
tests and C ABI sanitisation imply (ties, k > V, degenerate rows, NaN / inf,
padded and unaligned rows, out-of-range parameters).
"""
import glob
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - collected on CPU-only hosts too
    pytest.skip("no GPU", allow_module_level=True)

from mlxforge_amd import sampler, workloads  # noqa: E402
from tests import gpu_util as gu  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_config_parity(cfg):
    wl = workloads.make(cfg)
    say(f"[parity] config {cfg}: {wl.name}")
    dev = gu.to_device(wl.logits, wl.dtype)
    g = gu.gpu_sample(dev, T=wl.T, k=wl.k, p=wl.p, tlp=wl.tlp, u=wl.u, K_max=wl.K_max)
    o = gu.oracle_sample(wl.logits, wl.dtype, T=wl.T, k=wl.k, p=wl.p, tlp=wl.tlp, u=wl.u,
                         K_max=wl.K_max)
    rep = gu.compare(g, o, wl.dtype, tlp=wl.tlp, label=f"C{cfg}")
    say(f"[parity] config {cfg}: {rep}")
    # the stage count the host-side parameters call for gives the same results
    from mlxforge_amd import _lib
    code = {"f32": _lib.DTYPE_F32, "bf16": _lib.DTYPE_BF16, "f16": _lib.DTYPE_F16}[wl.dtype]
    st = _lib.refine_stages(wl.B, wl.V, code, wl.T, wl.k, wl.p)
    gh = gu.gpu_sample(dev, T=wl.T, k=wl.k, p=wl.p, tlp=wl.tlp, u=wl.u, K_max=wl.K_max, stages=st)
    for key in ("ids", "lp", "top_ids", "top_lp"):
        assert np.array_equal(g[key].view(np.uint32), gh[key].view(np.uint32)), \
            f"C{cfg}: {key} with {st} stages differs from 3"
    # determinism: a second run is bit-identical
    g2 = gu.gpu_sample(dev, T=wl.T, k=wl.k, p=wl.p, tlp=wl.tlp, u=wl.u, K_max=wl.K_max)
    assert np.array_equal(g["ids"], g2["ids"])
    assert np.array_equal(g["lp"].view(np.uint32), g2["lp"].view(np.uint32))


FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "fixtures", "*")))


@pytest.mark.parametrize("fx", FIXTURES, ids=[os.path.basename(f) for f in FIXTURES])
def test_real_logit_fixture_greedy(fx):
    logits = np.load(os.path.join(fx, "logits_last.npy"), allow_pickle=False)
    want = np.load(os.path.join(fx, "argmax.npy"), allow_pickle=False)
    dev = gu.to_device(logits, "f16")
    assert sampler.greedy(dev).cpu().numpy().tolist() == want.tolist()
    g = gu.gpu_sample(dev, tlp=[5], K_max=5)
    o = gu.oracle_sample(logits, "f16", tlp=[5], K_max=5)
    assert g["ids"].tolist() == want.tolist()
    gu.compare(g, o, "f16", tlp=[5], label=os.path.basename(fx))


def _rows(z):
    return torch.tensor(np.asarray(z, np.float32), device="cuda:0")


def test_known_answers():  # tests/sample/sampler_test.cpp
    # greedy (:41-44)
    assert sampler.greedy(_rows([[1, 3, 2], [5, 0, -1]])).tolist() == [1, 0]
    # T=0 is greedy (:46-52)
    P = sampler.SamplingParams
    r = sampler.Sampler.sample(_rows([[0.2, 0.9, 0.1, 0.4]]), P(temperature=0.0), [0.7])
    assert r.tokens.tolist() == [1]
    # ranked alternatives (:163-181)
    r = sampler.Sampler.sample(_rows([[1, 4, 2, 3, 0]]), P(temperature=0.0, top_logprobs=3), [0.0])
    assert r.top_tokens.tolist() == [[1, 3, 2]]
    assert r.tokens.tolist() == [1] and abs(r.logprobs.item() - r.top_logprobs[0, 0].item()) < 1e-6
    # full top-k normalised (:183-192)
    r = sampler.Sampler.sample(_rows([[0.5, 1.5, -0.5, 2.0]]), P(temperature=0.0, top_logprobs=4),
                               [0.0])
    assert abs(torch.exp(r.top_logprobs.double()).sum().item() - 1.0) < 1e-6
    # pre-temperature ordering (:194-203)
    r = sampler.Sampler.sample(_rows([[1, 4, 2, 3]]), P(temperature=0.8, top_logprobs=2), [0.5])
    assert r.top_tokens.tolist() == [[1, 3]]
    # top-p keeps {0,1} of probs (.5,.3,.15,.05) at p=.7 (:63-74): every u lands in them
    lg = np.log(np.array([0.5, 0.3, 0.15, 0.05], np.float32))
    for u in np.linspace(0.0, 0.999, 37):
        r = sampler.Sampler.sample(_rows([lg]), P(temperature=1.0, top_p=0.7), [float(u)])
        assert r.tokens.item() in (0, 1)
    # top-k=2 of distinct (5,1,4,2,3) keeps {0,2} (:54-61)
    for u in np.linspace(0.0, 0.999, 37):
        r = sampler.Sampler.sample(_rows([[5, 1, 4, 2, 3]]), P(temperature=1.0, top_k=2), [float(u)])
        assert r.tokens.item() in (0, 2)
    # same uniforms reproduce, different diverge (:126-134)
    z = torch.zeros(64, 16, device="cuda:0")
    u1 = torch.rand(64, generator=torch.Generator().manual_seed(42)).cuda()
    u2 = torch.rand(64, generator=torch.Generator().manual_seed(7)).cuda()
    a1 = sampler.Sampler.sample(z, P(), u1).tokens
    a2 = sampler.Sampler.sample(z, P(), u1).tokens
    b = sampler.Sampler.sample(z, P(), u2).tokens
    assert torch.equal(a1, a2) and not torch.equal(a1, b)
    assert torch.equal(a1.long(), (u1.double() * 16).floor().long())


def _random_case(rng, B, V, dtype):
    kind = rng.integers(0, 4)
    if kind == 0:
        z = rng.standard_normal((B, V)).astype(np.float32) * rng.uniform(0.05, 6)
    elif kind == 1:
        z = rng.integers(-3, 4, (B, V)).astype(np.float32)  # heavy ties
    elif kind == 2:
        z = (rng.gumbel(size=(B, V)) * 2).astype(np.float32)
    else:
        z = rng.standard_normal((B, V)).astype(np.float32) * 0.01
    if dtype == "bf16":
        host = workloads.to_bf16_bits(z)
    elif dtype == "f16":
        host = z.astype(np.float16)
    else:
        host = z
    T = np.where(rng.random(B) < 0.2, 0.0, rng.uniform(0.2, 2.0, B)).astype(np.float32)
    k = np.where(rng.random(B) < 0.5, rng.integers(1, V + 5, B), 0).astype(np.int32)
    p = np.where(rng.random(B) < 0.5, rng.uniform(0.05, 0.999, B), 1.0).astype(np.float32)
    tlp = rng.integers(-1, 6, B).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    return host, T, k, p, tlp, u


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("V", [1, 3, 7, 8, 9, 100, 2047, 2048, 2049, 5000, 33000])
def test_random_shapes(dtype, V):
    rng = np.random.default_rng(1000 + V + 7 * len(dtype))
    B = 1 if V > 20000 else 5
    host, T, k, p, tlp, u = _random_case(rng, B, V, dtype)
    K_max = min(5, V)
    say(f"[parity] random dtype={dtype} V={V} B={B}")
    g = gu.gpu_sample(gu.to_device(host, dtype), T=T, k=k, p=p, tlp=tlp, u=u, K_max=K_max)
    o = gu.oracle_sample(host, dtype, T=T, k=k, p=p, tlp=tlp, u=u, K_max=K_max)
    gu.compare(g, o, dtype, tlp=tlp, label=f"random {dtype} V={V}")


def test_padded_and_unaligned_rows():
    rng = np.random.default_rng(5)
    B, V = 6, 3001
    full = rng.standard_normal((B, V + 5)).astype(np.float32) * 3
    dev_full = torch.from_numpy(full).cuda()
    T = np.full(B, 0.9, np.float32)
    p = np.full(B, 0.8, np.float32)
    u = rng.random(B).astype(np.float32)
    tlp = np.full(B, 3, np.int32)
    # row_stride > V (bucket padding) and a 4-byte-offset view (scalar load path)
    for off in (0, 1):
        view = dev_full[:, off:off + V]
        host = np.ascontiguousarray(full[:, off:off + V])
        g = gu.gpu_sample(view, T=T, p=p, tlp=tlp, u=u, K_max=3)
        o = gu.oracle_sample(host, "f32", T=T, p=p, tlp=tlp, u=u, K_max=3)
        gu.compare(g, o, "f32", tlp=tlp, label=f"stride off={off}")


def test_degenerate_rows():
    V = 3000
    z = np.zeros((6, V), np.float32)
    z[0] = -np.inf                       # all masked
    z[1, ::7] = np.nan                   # NaN reads as -inf
    z[2, 5] = np.inf
    z[2, 2000] = np.inf                  # two +inf entries share the mass
    z[3] = 1.0                           # constant row: every entry ties
    z[4, 1234] = 7.0
    z[4, 2345] = 7.0                     # duplicate maximum
    z[5] = np.linspace(-5, 5, V, dtype=np.float32)
    host = z
    T = np.array([1.0, 1.0, 1.0, 1.0, 0.0, 1.0], np.float32)
    k = np.array([0, 3, 0, 10, 0, 1], np.int32)
    p = np.array([0.5, 0.9, 1.0, 0.3, 1.0, 1.0], np.float32)
    tlp = np.array([0, 2, 2, 4, 3, 1], np.int32)
    for u in (0.0, 0.37, 0.999999):
        uu = np.full(6, u, np.float32)
        g = gu.gpu_sample(gu.to_device(host, "f32"), T=T, k=k, p=p, tlp=tlp, u=uu, K_max=4)
        o = gu.oracle_sample(host, "f32", T=T, k=k, p=p, tlp=tlp, u=uu, K_max=4)
        gu.compare(g, o, "f32", tlp=tlp, label=f"degenerate u={u}")
    assert g["ids"][4] == 1234


# (B, V) shapes that select each first-pass slice layout: 32, 16 and 8 logits
# per thread of a 256-thread slice
LAYOUT_SHAPES = [(32, 151936), (8, 151936), (1, 128256)]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("B,V", LAYOUT_SHAPES)
def test_degenerate_rows_each_layout(B, V, dtype):
    """Constant rows (the heavy-tie fallback of the per-slice best-64 list),
    all -inf, NaN stripes, two +inf, duplicate maxima, each with a list-using
    parameter set, in every slice layout."""
    rng = np.random.default_rng(77 + B)
    z = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    kinds = B if B < 6 else 6
    for r in range(B):
        c = r % 6 if kinds == 6 else 3
        if c == 0:
            z[r] = -np.inf
        elif c == 1:
            z[r, ::5] = np.nan
        elif c == 2:
            z[r, 7] = np.inf
            z[r, V - 3] = np.inf
        elif c == 3:
            z[r] = 0.5
        elif c == 4:
            z[r, 100] = 30.0
            z[r, V - 100] = 30.0
    host = z if dtype == "f32" else workloads.to_bf16_bits(z)
    T = rng.choice(np.array([0.0, 0.8, 1.0], np.float32), B).astype(np.float32)
    k = rng.choice(np.array([0, 1, 5, 40], np.int32), B).astype(np.int32)
    p = rng.choice(np.array([1.0, 0.9], np.float32), B).astype(np.float32)
    tlp = rng.choice(np.array([0, 3, 5], np.int32), B).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    say(f"[parity] degenerate layout B={B} V={V} {dtype}")
    g = gu.gpu_sample(gu.to_device(host, dtype), T=T, k=k, p=p, tlp=tlp, u=u, K_max=5)
    o = gu.oracle_sample(host, dtype, T=T, k=k, p=p, tlp=tlp, u=u, K_max=5)
    gu.compare(g, o, dtype, tlp=tlp, label=f"degenerate layout B={B} V={V} {dtype}")


# quiet and signalling NaNs of both signs, as bit patterns of each dtype
NAN_BITS = {"f32": [0x7fc00000, 0xffc00000, 0x7f800001, 0xff800001],
            "bf16": [0x7fc0, 0xffc0, 0x7f81, 0xff81],
            "f16": [0x7e00, 0xfe00, 0x7c01, 0xfc01]}


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_nan_patterns_every_path(dtype):
    """Every NaN bit pattern reads as -inf on every row kind: scattered NaNs,
    a NaN where the row maximum was, and a whole slice of NaNs."""
    rng = np.random.default_rng(31)
    B, V = 8, 20000
    z = rng.standard_normal((B, V)).astype(np.float32) * np.float32(2.0)
    if dtype == "f32":
        bits = z.view(np.uint32).copy()
    elif dtype == "bf16":
        bits = workloads.to_bf16_bits(z)
    else:
        bits = z.astype(np.float16).view(np.uint16).copy()
    nb = np.array(NAN_BITS[dtype], dtype=bits.dtype)
    for r in range(B):
        pos = rng.choice(V, 40, replace=False)
        bits[r, pos] = nb[np.arange(40) % 4]
    bits[0, int(np.argmax(z[0]))] = nb[1]
    bits[7, 8192:16384] = nb[2]
    host = bits.view(np.float32) if dtype == "f32" else (bits.view(np.float16) if dtype == "f16" else bits)
    T = np.array([0.0, 1.0, 0.7, 1.0, 0.9, 1.0, 1.2, 1.0], np.float32)
    k = np.array([0, 5, 0, 200, 0, 40, 0, 0], np.int32)
    p = np.array([1.0, 1.0, 0.9, 0.95, 1.0, 0.8, 1.0, 0.9], np.float32)
    tlp = np.array([2, 0, 3, -1, 1, 5, 0, 2], np.int32)
    u = rng.random(B).astype(np.float32)
    g = gu.gpu_sample(gu.to_device(host, dtype), T=T, k=k, p=p, tlp=tlp, u=u, K_max=5)
    o = gu.oracle_sample(host, dtype, T=T, k=k, p=p, tlp=tlp, u=u, K_max=5)
    gu.compare(g, o, dtype, tlp=tlp, label=f"NaN patterns {dtype}")


def test_parameter_sanitisation():
    rng = np.random.default_rng(9)
    V = 4000
    z = (rng.standard_normal((8, V)) * 2).astype(np.float32)
    T = np.array([np.nan, np.inf, -1.0, 0.0, 1e-30, 1.0, 1.0, 1.0], np.float32)
    k = np.array([0, 0, 0, 0, 0, 10 ** 6, -5, 1], np.int32)
    p = np.array([1.0, 1.0, 1.0, 1.0, 1.0, 1e-7, 1.5, np.nan], np.float32)
    u = np.array([0.5, 0.5, 0.5, 0.5, 0.5, -3.0, 7.0, np.nan], np.float32)
    tlp = np.zeros(8, np.int32)
    g = gu.gpu_sample(gu.to_device(z, "f32"), T=T, k=k, p=p, tlp=tlp, u=u)
    o = gu.oracle_sample(z, "f32", T=T, k=k, p=p, tlp=tlp, u=u)
    gu.compare(g, o, "f32", tlp=tlp, label="sanitisation")


def test_large_candidate_sets():
    # top-p over a flat row: the boundary bin holds far more candidates than LDS
    rng = np.random.default_rng(11)
    V = 60000
    z = np.zeros((3, V), np.float32)
    z[1] = rng.integers(0, 2, V).astype(np.float32) * 1e-3
    z[2] = (rng.standard_normal(V) * 1e-4).astype(np.float32)
    T = np.ones(3, np.float32)
    p = np.array([0.5, 0.7, 0.95], np.float32)
    k = np.array([0, 40000, 0], np.int32)
    u = np.array([0.3, 0.6, 0.9], np.float32)
    for dtype in ("f32", "bf16"):
        host = z if dtype == "f32" else workloads.to_bf16_bits(z)
        g = gu.gpu_sample(gu.to_device(host, dtype), T=T, k=k, p=p, u=u)
        o = gu.oracle_sample(host, dtype, T=T, k=k, p=p, u=u)
        gu.compare(g, o, dtype, label=f"large candidates {dtype}")


def test_workspace_reuse_across_shapes():
    """One workspace serves calls of different shapes in a row: B grows (the
    per-row counters must still read zero), then shrinks, then grows again."""
    ws = sampler.Workspace("cuda:0")
    rng = np.random.default_rng(77)
    for B, V, dtype in [(2, 3000, "bf16"), (40, 3000, "bf16"), (3, 20000, "f32"), (70, 5000, "f16"),
                        (2, 3000, "bf16")]:
        host, T, k, p, tlp, u = _random_case(rng, B, V, dtype)
        p = np.where(rng.random(B) < 0.7, rng.uniform(0.3, 0.99, B), p).astype(np.float32)
        k = np.where(p < 1.0, 0, k).astype(np.int32)  # mostly top-p-only rows
        say(f"[parity] workspace reuse B={B} V={V} {dtype}")
        dev = gu.to_device(host, dtype)
        f = lambda a, t: torch.as_tensor(np.asarray(a), dtype=t).to("cuda:0")
        res = sampler.sample_rows(dev, temperature=f(T, torch.float32), top_k=f(k, torch.int32),
                                  top_p=f(p, torch.float32), top_logprobs=f(tlp, torch.int32),
                                  uniforms=f(u, torch.float32), K_max=3, workspace=ws)
        torch.cuda.synchronize()
        g = dict(ids=res.tokens.cpu().numpy(), lp=res.logprobs.cpu().numpy(),
                 top_ids=res.top_tokens.cpu().numpy(), top_lp=res.top_logprobs.cpu().numpy())
        o = gu.oracle_sample(host, dtype, T=T, k=k, p=p, tlp=tlp, u=u, K_max=3)
        gu.compare(g, o, dtype, tlp=tlp, label=f"workspace reuse B={B} V={V} {dtype}")


def test_workspace_errors():
    from mlxforge_amd import _lib
    z = torch.zeros(2, 100, device="cuda:0")
    ws = sampler.Workspace("cuda:0")
    ws.buf = torch.empty(16, dtype=torch.uint8, device="cuda:0")
    ids = torch.empty(2, dtype=torch.int32, device="cuda:0")
    import ctypes
    err = ctypes.c_void_p()
    rc = _lib.load().mlxf_greedy(ctypes.c_void_p(z.data_ptr()), 0, 2, 100, 100,
                                 ctypes.c_void_p(ids.data_ptr()), ctypes.c_void_p(ws.buf.data_ptr()),
                                 16, None, ctypes.byref(err))
    assert rc == _lib.EWORKSPACE
    _lib.load().mlxf_string_free(err)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_stage_counts_agree(dtype):
    """Rows still open after the last refine stage launched are finished by its
    deciding kernel: every stage count gives bit-identical results."""
    rng = np.random.default_rng(77 + len(dtype))
    for V in (3000, 20000):
        host, T, k, p, tlp, u = _random_case(rng, 6, V, dtype)
        dev = gu.to_device(host, dtype)
        say(f"[parity] stage counts dtype={dtype} V={V}")
        ref = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u, K_max=3, stages=3)
        o = gu.oracle_sample(host, dtype, T=T, k=k, p=p, tlp=tlp, u=u, K_max=3)
        gu.compare(ref, o, dtype, tlp=tlp, label=f"stages {dtype} V={V}")
        for st in (0, 1, 2):
            g = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u, K_max=3, stages=st)
            assert np.array_equal(g["ids"], ref["ids"]), (st, g["ids"], ref["ids"])
            assert np.array_equal(g["lp"].view(np.uint32), ref["lp"].view(np.uint32))


def _minp_case(rng, B, V, dtype, kind):
    """Rows where min_p binds or not, behind each earlier filter: temperature
    only, top-k <= 63, top-k > 63, top-p, and top-k > 63 with top-p."""
    z = rng.standard_normal((B, V)).astype(np.float32) * np.float32(rng.uniform(0.5, 3.0))
    for r in range(B):
        hot = rng.choice(V, size=min(V, 12), replace=False)
        z[r, hot] += rng.uniform(2.0, 6.0, hot.size).astype(np.float32)
    host = z if dtype == "f32" else (workloads.to_bf16_bits(z) if dtype == "bf16" else z.astype(np.float16))
    T = rng.uniform(0.4, 1.3, B).astype(np.float32)
    k = np.zeros(B, np.int32)
    p = np.ones(B, np.float32)
    if kind in ("klist",):
        k[:] = rng.integers(1, 60, B)
    if kind in ("khist", "khist_topp"):
        k[:] = rng.integers(100, 3000, B)
    if kind in ("topp", "khist_topp"):
        p[:] = rng.uniform(0.5, 0.99, B)
    mp = rng.choice(np.array([0.0, 0.001, 0.02, 0.1, 0.3, 0.7, 1.0], np.float32), B)
    tlp = rng.integers(-1, 3, B).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    return host, T, k, p, mp, tlp, u


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("kind", ["temp", "klist", "khist", "topp", "khist_topp"])
def test_min_p_parity(dtype, kind):
    """min_p (src/sample/sampler.cpp:87-93, after top-p) against the oracle,
    behind every earlier filter, at every refine stage count."""
    rng = np.random.default_rng(500 + len(kind) * 13 + len(dtype))
    for V in (4000, 30000):
        B = 8
        host, T, k, p, mp, tlp, u = _minp_case(rng, B, V, dtype, kind)
        say(f"[parity] min_p {kind} dtype={dtype} V={V}")
        dev = gu.to_device(host, dtype)
        o = gu.oracle_sample(host, dtype, T=T, k=k, p=p, tlp=tlp, u=u, K_max=2, min_p=mp)
        ref = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u, K_max=2, min_p=mp, stages=3)
        gu.compare(ref, o, dtype, tlp=tlp, label=f"min_p {kind} {dtype} V={V}")
        for st in (0, 1):
            g = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u, K_max=2, min_p=mp, stages=st)
            assert np.array_equal(g["ids"], ref["ids"]), (kind, st, g["ids"], ref["ids"])


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_min_p_one_draws_the_max(dtype):
    """min_p = 1 keeps only the row max and its ties, behind every earlier
    filter: the id is the argmax (one max) or one of the tied maxima, whatever
    the uniform -- checked directly, not through the oracle."""
    rng = np.random.default_rng(1234 + len(dtype))
    B, V = 16, 30000
    z = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    ties = {}
    for r in range(B):
        top = float(np.float32(z[r].max() + 3.0))
        if r % 2:
            pos = rng.choice(V, size=int(rng.integers(2, 6)), replace=False)
        else:
            pos = rng.choice(V, size=1)
        z[r, pos] = top
        ties[r] = set(int(i) for i in pos)
    host = z if dtype == "f32" else (workloads.to_bf16_bits(z) if dtype == "bf16" else z.astype(np.float16))
    vals = gu.host_values(host, dtype)
    for r in range(B):  # the tie set in the dtype's own values
        ties[r] = set(np.nonzero(vals[r] == vals[r].max())[0].tolist())
    T = rng.uniform(0.5, 1.5, B).astype(np.float32)
    k = np.array([0, 0, 5, 5, 200, 200, 0, 0] * 2, np.int32)
    p = np.array([1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 0.9, 0.9] * 2, np.float32)
    mp = np.ones(B, np.float32)
    dev = gu.to_device(host, dtype)
    for u in (0.0, 0.3, 0.7, 0.9999):
        uu = np.full(B, u, np.float32)
        for st in (0, 3):
            g = gu.gpu_sample(dev, T=T, k=k, p=p, u=uu, min_p=mp, stages=st)
            for r in range(B):
                assert int(g["ids"][r]) in ties[r], (dtype, u, st, r, g["ids"][r], sorted(ties[r]))


def _mixed_rows(rng, B, V, dtype):
    """Rows of every kind at once: flat, peaked, heavy ties, -inf runs."""
    z = np.empty((B, V), np.float32)
    for r in range(B):
        kind = r % 4
        if kind == 0:    # flat: few distinct 16-bit values, many ties
            z[r] = np.round(rng.standard_normal(V) * 0.1, 2)
        elif kind == 1:  # peaked
            z[r] = rng.standard_normal(V) * 3
            z[r, rng.integers(0, V, 5)] += 12
        elif kind == 2:  # ties at the top
            z[r] = rng.standard_normal(V)
            z[r, rng.integers(0, V, 200)] = z[r].max() + 1
        else:            # masked-out runs
            z[r] = rng.standard_normal(V) * 2
            z[r, : V // 3] = -np.inf
    if dtype == "f32":
        host = z
    elif dtype == "bf16":
        host = workloads.to_bf16_bits(np.nan_to_num(z, neginf=-3e38))
        host[np.isneginf(z)] = 0xFF80
    else:
        host = z.astype(np.float16)
    T = rng.choice(np.array([0.0, 0.5, 1.0, 1.7], np.float32), B)
    k = rng.choice(np.array([0, 0, 1, 10, 63, 64, 500, 5000], np.int32), B)
    p = rng.choice(np.array([1.0, 1.0, 0.3, 0.9, 0.999], np.float32), B)
    mp = rng.choice(np.array([0.0, 0.0, 0.01, 0.2, 0.9], np.float32), B)
    tlp = rng.integers(-1, 4, B).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    return host, T, k, p, mp, tlp, u


@pytest.mark.parametrize("seed", range(6))
def test_mixed_rows_every_path(seed):
    """Every row kind and parameter combination in one call, all three dtypes,
    at the generic and the hinted stage count."""
    rng = np.random.default_rng(7000 + seed)
    dtype = ("f32", "bf16", "f16")[seed % 3]
    V = int(rng.integers(1000, 70000))
    B = 16
    host, T, k, p, mp, tlp, u = _mixed_rows(rng, B, V, dtype)
    say(f"[parity] mixed rows seed={seed} dtype={dtype} V={V}")
    dev = gu.to_device(host, dtype)
    o = gu.oracle_sample(host, dtype, T=T, k=k, p=p, tlp=tlp, u=u, K_max=3, min_p=mp)
    g = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u, K_max=3, min_p=mp)
    gu.compare(g, o, dtype, tlp=tlp, label=f"mixed seed={seed}")
    gh = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u, K_max=3, min_p=mp, stages=1)
    assert np.array_equal(gh["ids"], g["ids"])


def _peaked_topp_case(rng, B, V, dtype):
    """Top-p rows whose nucleus mostly lies in the best 64 (Zipf-like and
    spiked rows), with some whose nucleus does not (flat rows), exact ties at
    the top (values on a 0.5 grid), temperatures from 0.05 to 2, and min_p."""
    z = np.empty((B, V), np.float32)
    for r in range(B):
        kind = r % 5
        if kind == 0:
            z[r] = rng.gumbel(size=V) * 2.5 - 1.1 * np.log(np.arange(1, V + 1))
        elif kind == 1:
            z[r] = rng.standard_normal(V) * 0.5
            hot = rng.choice(V, size=min(V, 20), replace=False)
            z[r, hot] += rng.uniform(4.0, 12.0, hot.size)
        elif kind == 2:
            z[r] = np.round(rng.standard_normal(V) * 2, 0) * 0.5 - 3.0
            z[r, rng.choice(V, size=min(V, 40), replace=False)] = 4.0  # a tie group at the top
        elif kind == 3:
            z[r] = rng.standard_normal(V) * 0.2  # flat: the nucleus is far beyond the list
        else:
            z[r] = rng.gumbel(size=V) * 4.0
    host = z if dtype == "f32" else (workloads.to_bf16_bits(z) if dtype == "bf16" else z.astype(np.float16))
    T = rng.choice(np.array([0.05, 0.3, 0.7, 1.0, 1.6, 2.0], np.float32), B)
    k = np.zeros(B, np.int32)
    p = rng.choice(np.array([0.1, 0.5, 0.8, 0.9, 0.95, 0.99, 0.999], np.float32), B)
    mp = rng.choice(np.array([0.0, 0.0, 0.0, 0.01, 0.2], np.float32), B)
    u = rng.random(B).astype(np.float32)
    return host, T, k, p, mp, u


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("V", [100, 5000, 151936])
def test_topp_from_best_list(dtype, V):
    """Top-p rows that want top_logprobs (so carry a best-64 list) are
    finished in the first deciding kernel when the bounds on the row's total
    mass put the nucleus inside the list; every other row takes the refine
    stages.  Both must agree with the oracle, and every stage count (0: rows
    the list cannot settle are finished serially) must give the same bits.
    A third of the rows want no alternatives (no list: the stages)."""
    rng = np.random.default_rng(2024 + V + len(dtype))
    B = 20
    host, T, k, p, mp, u = _peaked_topp_case(rng, B, V, dtype)
    tlp = np.full(B, 3, np.int32)
    tlp[::3] = 0
    K_max = 3
    dev = gu.to_device(host, dtype)
    say(f"[parity] top-p from the best list dtype={dtype} V={V}")
    ref = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u, K_max=K_max, stages=3, min_p=mp)
    o = gu.oracle_sample(host, dtype, T=T, k=k, p=p, tlp=tlp, u=u, K_max=K_max, min_p=mp)
    rep = gu.compare(ref, o, dtype, tlp=tlp, label=f"topp list {dtype} V={V}")
    say(f"[parity] {rep}")
    for st in (0, 1, 2):
        g = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u, K_max=K_max, stages=st, min_p=mp)
        assert np.array_equal(g["ids"], ref["ids"]), (st, g["ids"], ref["ids"])
        assert np.array_equal(g["lp"].view(np.uint32), ref["lp"].view(np.uint32))
