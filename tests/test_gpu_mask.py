"""GPU parity of the grammar-constrained rows (src/runtime/worker.cpp:142-179,
455-459): the bit-masked fp32 rows bit-exact against the oracle's row + fp32
mask, and sampling them as fp32 logits against the oracle."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - collected on CPU-only hosts too
    pytest.skip("no GPU", allow_module_level=True)

from mlxforge_amd import sampler, workloads  # noqa: E402
from oracle import oracle as orc  # noqa: E402
from tests import gpu_util as gu  # noqa: E402


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("V", [33, 4097, 151936])
def test_mask_matches_oracle_and_samples(dtype, V):
    rng = np.random.default_rng(60 + V + len(dtype))
    B = 6
    z = (rng.standard_normal((B, V)) * 3).astype(np.float32)
    host = z if dtype == "f32" else (workloads.to_bf16_bits(z) if dtype == "bf16" else z.astype(np.float16))
    vals = workloads.bf16_bits_to_f32(host) if dtype == "bf16" else host.astype(np.float32)
    allowed = rng.random((B, V)) < np.array([0.5, 0.01, 1.0, 0.0, 0.2, 0.9])[:, None]
    allowed[1, :] = False
    allowed[1, rng.integers(0, V)] = True  # a single allowed token
    print(f"[mask] dtype={dtype} V={V}", flush=True)
    bits = torch.from_numpy(orc.pack_bits(allowed).view(np.int32)).cuda()
    out = sampler.apply_mask(gu.to_device(host, dtype), bits)
    torch.cuda.synchronize()
    exp = np.stack([orc.apply_mask(vals[r], allowed[r]) for r in range(B)])
    assert np.array_equal(out.cpu().numpy().view(np.uint32), exp.view(np.uint32))
    T = np.array([0.0, 1.0, 0.8, 1.0, 1.2, 0.7], np.float32)
    k = np.array([0, 0, 30, 0, 0, 200], np.int32)
    p = np.array([1.0, 0.9, 1.0, 0.95, 1.0, 0.9], np.float32)
    u = rng.random(B).astype(np.float32)
    tlp = np.zeros(B, np.int32)
    g = gu.gpu_sample(out, T=T, k=k, p=p, tlp=tlp, u=u)
    o = gu.oracle_sample(exp, "f32", T=T, k=k, p=p, tlp=tlp, u=u)
    gu.compare(g, o, "f32", tlp=tlp, label=f"masked {dtype} V={V}")
    ids = g["ids"]
    for r in range(B):
        if allowed[r].any():
            assert allowed[r, ids[r]], (r, ids[r])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_mask_strided_and_unaligned_rows(dtype):
    """Padded rows (row, bit-mask and output strides beyond V) and row starts
    that are not 16-byte aligned take the element-wise loads and stores."""
    rng = np.random.default_rng(7 + len(dtype))
    B, V = 5, 10007
    nw = (V + 31) // 32
    z = (rng.standard_normal((B, V + 3)) * 3).astype(np.float32)
    host = z if dtype == "f32" else workloads.to_bf16_bits(z)
    vals = workloads.bf16_bits_to_f32(host) if dtype == "bf16" else host.astype(np.float32)
    allowed = rng.random((B, V)) < np.array([0.3, 0.0, 1.0, 0.001, 0.7])[:, None]
    packed = orc.pack_bits(allowed).view(np.int32)
    bits = torch.zeros((B, nw + 5), dtype=torch.int32, device="cuda")
    bits[:, :nw] = torch.from_numpy(packed).cuda()
    bits[:, nw:] = -1  # words past the row's own must not count
    for off in (0, 1):  # off = 1: rows start one element in (not 16-byte aligned)
        print(f"[mask strided] dtype={dtype} offset={off}", flush=True)
        dev = gu.to_device(host, dtype)[:, off:off + V]
        out_full = torch.full((B, V + 9), 7.0, dtype=torch.float32, device="cuda")
        out = out_full[:, 1:1 + V] if off else out_full[:, :V]
        sampler.apply_mask(dev, bits, V=V, out=out)
        torch.cuda.synchronize()
        exp = np.stack([orc.apply_mask(vals[r, off:off + V], allowed[r]) for r in range(B)])
        assert np.array_equal(out.cpu().numpy().view(np.uint32), exp.view(np.uint32))
        full = out_full.cpu().numpy()
        lo = 1 if off else 0
        assert (full[:, :lo] == 7.0).all() and (full[:, lo + V:] == 7.0).all()  # nothing written outside
