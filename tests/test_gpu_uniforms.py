"""GPU parity of the device draw uniforms (Philox4x32-10 keyed by the row
seed at counter step) against the oracle's restatement, and the reference's
reproducibility property (tests/sample/sampler_test.cpp:126-134) end to end."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - collected on CPU-only hosts too
    pytest.skip("no GPU", allow_module_level=True)

from mlxforge_amd import sampler  # noqa: E402
from oracle import oracle as orc  # noqa: E402


def test_uniforms_match_oracle():
    rng = np.random.default_rng(3)
    B = 1000
    seeds = rng.integers(0, 2**63, B, dtype=np.int64).astype(np.uint64)
    seeds[:3] = [0, 2**64 - 1, 2**63]
    steps = rng.integers(0, 2**40, B, dtype=np.int64).astype(np.uint64)
    print("[uniforms] per-row steps and a shared step", flush=True)
    sd = torch.from_numpy(seeds.view(np.int64)).cuda()
    g = sampler.uniforms(sd, torch.from_numpy(steps.view(np.int64)).cuda())
    assert np.array_equal(g.cpu().numpy().view(np.uint32), orc.uniforms(seeds, steps).view(np.uint32))
    g2 = sampler.uniforms(sd, 12345)
    assert np.array_equal(g2.cpu().numpy().view(np.uint32), orc.uniforms(seeds, 12345).view(np.uint32))


def test_seeded_sampling_replays():
    """Same seed and step: same tokens; the next step draws anew."""
    rng = np.random.default_rng(8)
    B, V = 64, 5000
    z = torch.from_numpy((rng.standard_normal((B, V)) * 2).astype(np.float32)).cuda()
    sd = torch.arange(B, dtype=torch.int64, device="cuda") * 7919
    toks = []
    for step in (5, 5, 6):
        u = sampler.uniforms(sd, step)
        toks.append(sampler.sample_rows(z, temperature=1.0, uniforms=u).tokens.cpu().numpy())
    assert np.array_equal(toks[0], toks[1])
    assert not np.array_equal(toks[0], toks[2])
