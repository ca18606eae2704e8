"""GPU parity of top_logprobs wider than the sampling kernels' best-64 lists
(top_k_logprobs, src/sample/sampler.cpp:30-38, K = min(top_logprobs, V) at
:52): calls with K_max above 64 against the oracle, ids exact (ties by lowest
index) and logprobs within tolerance, with the sampled ids and chosen
logprobs of the same call checked as usual."""
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


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("V,K_max", [(1000, 65), (1000, 1000), (50001, 200), (151936, 4096)])
def test_wide_top_logprobs(dtype, V, K_max):
    rng = np.random.default_rng(300 + V + K_max + len(dtype))
    B = 10
    z = np.empty((B, V), np.float32)
    for r in range(B):
        if r % 3 == 0:
            z[r] = rng.standard_normal(V) * 4
        elif r % 3 == 1:
            z[r] = np.round(rng.standard_normal(V) * 2, 1)  # many ties across the K-th entry
        else:
            z[r] = rng.gumbel(size=V) * 2.5 - 1.1 * np.log(np.arange(1, V + 1))
    host = z if dtype == "f32" else (workloads.to_bf16_bits(z) if dtype == "bf16" else z.astype(np.float16))
    tlp = np.array([K_max, -1, 0, 1, 20, 64, 65, K_max // 2 + 1, K_max, 10 ** 6], np.int32)[:B]
    T = np.array([1.0, 0.0, 0.7, 1.0, 1.3, 0.9, 1.0, 1.1, 0.0, 1.0], np.float32)[:B]
    k = np.array([0, 0, 50, 0, 5, 0, 1000, 0, 0, 0], np.int32)[:B]
    p = np.array([0.9, 1.0, 1.0, 0.95, 1.0, 0.8, 1.0, 1.0, 1.0, 0.5], np.float32)[:B]
    u = rng.random(B).astype(np.float32)
    say(f"[topk-wide] dtype={dtype} V={V} K_max={K_max}")
    dev = gu.to_device(host, dtype)
    g = gu.gpu_sample(dev, T=T, k=k, p=p, tlp=tlp, u=u, K_max=K_max, stages=2)
    o = gu.oracle_sample(host, dtype, T=T, k=k, p=p, tlp=tlp, u=u, K_max=K_max)
    gu.compare(g, o, dtype, tlp=tlp, label=f"wide K={K_max}")
    # rows with top_logprobs < 1 or beyond K_max: the columns past the row's K
    Kr = np.minimum(np.where(tlp > 0, tlp, 0), min(K_max, V))
    for r in range(B):
        assert (g["top_ids"][r, Kr[r]:] == -1).all() and np.isneginf(g["top_lp"][r, Kr[r]:]).all()
