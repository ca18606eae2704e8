"""GPU parity of the penalties (src/sample/sampler.cpp:95-133) through the C
ABI: the logits penalized in place must equal the oracle's, bit for bit, and
sampling the penalized logits must match the oracle on the same logits."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - collected on CPU-only hosts too
    pytest.skip("no GPU", allow_module_level=True)

from mlxforge_amd import sampler, workloads  # noqa: E402
from oracle import oracle as orc  # noqa: E402
from tests import gpu_util as gu  # noqa: E402


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _host_values(host, dtype):
    if dtype == "bf16":
        return workloads.bf16_bits_to_f32(host)
    return host.astype(np.float32)


def _case(rng, B, V, N, dtype):
    z = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
    z[0, : min(V, 5)] = 0.0  # zeros and ties among the history ids
    host = z if dtype == "f32" else (workloads.to_bf16_bits(z) if dtype == "bf16" else z.astype(np.float16))
    hist = rng.integers(-3, V + 3, (B, N)).astype(np.int32)  # a few ids out of range
    hot = rng.integers(0, V, (B, 8))
    for r in range(B):  # repeated ids (counts up to ~40)
        hist[r, : N // 2] = hot[r, rng.integers(0, 8, N // 2)]
    hl = rng.integers(0, N + 1, B).astype(np.int32)
    rep = rng.choice(np.array([1.0, 1.3, 0.8, 4.0, np.nan, -1.0], np.float32), B)
    fq = rng.choice(np.array([0.0, 0.25, -0.5, 1.0], np.float32), B)
    ps = rng.choice(np.array([0.0, 0.7, -0.3], np.float32), B)
    return host, hist, hl, rep, fq, ps


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("V,N", [(50, 64), (5000, 300), (40000, 3000)])
def test_penalties_match_oracle(dtype, V, N):
    rng = np.random.default_rng(900 + V + N + len(dtype))
    B = 12
    host, hist, hl, rep, fq, ps = _case(rng, B, V, N, dtype)
    say(f"[penalties] dtype={dtype} V={V} N={N}")
    dev = gu.to_device(host, dtype)
    sampler.apply_penalties(dev, torch.from_numpy(hist).cuda(), hist_len=hl, repetition=rep,
                            frequency=fq, presence=ps)
    torch.cuda.synchronize()
    got = dev.float().cpu().numpy()
    vals = _host_values(host, dtype)
    code = gu.DT[dtype][1]
    for r in range(B):
        exp = orc.apply_penalties(vals[r], hist[r, : hl[r]], rep=float(rep[r]), freq=float(fq[r]),
                                  pres=float(ps[r]), dtype=code)
        assert np.array_equal(got[r].view(np.uint32), exp.view(np.uint32)), (r, rep[r], fq[r], ps[r])
    # a second call on fresh logits: the counters were left at zero
    dev2 = gu.to_device(host, dtype)
    sampler.apply_penalties(dev2, torch.from_numpy(hist).cuda(), hist_len=hl, repetition=rep,
                            frequency=fq, presence=ps)
    torch.cuda.synchronize()
    assert np.array_equal(dev2.float().cpu().numpy().view(np.uint32), got.view(np.uint32))


def test_penalized_sampling_matches_oracle():
    """Penalties then sampling (greedy rows too: src/sample/sampler.cpp:141-156)."""
    rng = np.random.default_rng(17)
    B, V, N = 16, 20000, 500
    host, hist, hl, rep, fq, ps = _case(rng, B, V, N, "bf16")
    T = rng.choice(np.array([0.0, 0.7, 1.0], np.float32), B)
    k = rng.choice(np.array([0, 20, 200], np.int32), B)
    p = rng.choice(np.array([1.0, 0.9], np.float32), B)
    u = rng.random(B).astype(np.float32)
    tlp = np.zeros(B, np.int32)
    dev = gu.to_device(host, "bf16")
    sampler.apply_penalties(dev, torch.from_numpy(hist).cuda(), hist_len=hl, repetition=rep,
                            frequency=fq, presence=ps)
    g = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u)
    vals = workloads.bf16_bits_to_f32(host)
    adj = np.stack([orc.apply_penalties(vals[r], hist[r, : hl[r]], rep=float(rep[r]), freq=float(fq[r]),
                                        pres=float(ps[r]), dtype=orc.BF16) for r in range(B)])
    o = gu.oracle_sample(workloads.to_bf16_bits(adj), "bf16", T=T, k=k, p=p, tlp=tlp, u=u)
    gu.compare(g, o, "bf16", tlp=tlp, label="penalized sampling")
