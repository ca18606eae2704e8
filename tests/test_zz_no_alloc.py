"""mlxf_sample_noalloc, the entry point that allocates nothing, through the C
ABI: its results equal mlxf_sample_ex's on the same inputs, bit for bit (the
same kernels, with the library's fixed per-GPU scratch in place of the
caller's workspace), on two calls in a row, the second with a smaller input;
a shape whose workspace exceeds the scratch is refused."""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - collected on CPU-only hosts too
    pytest.skip("no GPU", allow_module_level=True)

from mlxforge_amd import _lib, workloads  # noqa: E402

P = ctypes.c_void_p


def _inputs(rng, B, V, dtype):
    z = (rng.standard_normal((B, V)) * rng.uniform(0.1, 3.0)).astype(np.float32)
    host = workloads.to_bf16_bits(z) if dtype == "bf16" else z
    t = (torch.from_numpy(host.view(np.int16)).view(torch.bfloat16) if dtype == "bf16"
         else torch.from_numpy(host)).to("cuda:0")
    f = lambda a, ty: torch.as_tensor(a, dtype=ty).to("cuda:0")
    T = f(np.where(rng.random(B) < 0.2, 0.0, rng.uniform(0.5, 1.3, B)), torch.float32)
    k = f(rng.choice([0, 0, 5, 40, 300], B), torch.int32)
    p = f(rng.choice([1.0, 0.9, 0.6], B), torch.float32)
    mp = f(rng.choice([0.0, 0.0, 0.05], B), torch.float32)
    tlp = f(rng.integers(-1, 4, B), torch.int32)
    u = f(rng.random(B), torch.float32)
    return t, T, k, p, mp, tlp, u


def _outs(B, K):
    d = "cuda:0"
    return (torch.full((B,), -7, dtype=torch.int32, device=d), torch.full((B,), 7.0, device=d),
            torch.full((B, K), -7, dtype=torch.int32, device=d), torch.full((B, K), 7.0, device=d))


def _call(noalloc, t, code, B, V, T, k, p, mp, tlp, u, K, stages, ws=None):
    L = _lib.load()
    ids, lp, tid, tlpv = _outs(B, K)
    err = P()
    stream = P(torch.cuda.current_stream().cuda_stream)
    args = [P(t.data_ptr()), code, B, V, V, P(T.data_ptr()), P(k.data_ptr()), P(p.data_ptr()),
            P(mp.data_ptr()), P(tlp.data_ptr()), P(u.data_ptr()), P(ids.data_ptr()), P(lp.data_ptr()),
            P(tid.data_ptr()), P(tlpv.data_ptr()), K]
    if noalloc:
        rc = L.mlxf_sample_noalloc(*args, stages, stream, ctypes.byref(err))
    else:
        rc = L.mlxf_sample_ex(*args, P(ws.data_ptr()), ws.numel(), stages, stream, ctypes.byref(err))
    _lib.check(rc, err)
    torch.cuda.synchronize()
    return [x.cpu().numpy() for x in (ids, lp, tid, tlpv)]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_noalloc_matches_workspace_entry(dtype):
    rng = np.random.default_rng(2024 + len(dtype))
    code = _lib.DTYPE_F32 if dtype == "f32" else _lib.DTYPE_BF16
    K = 4
    # a large call, then a smaller one: the scratch keeps the first call's
    # contents, which the second must not depend on
    for B, V in ((64, 151936), (5, 3001)):
        print(f"[noalloc] {dtype} B={B} V={V}", flush=True)
        sys.stdout.flush()
        t, T, k, p, mp, tlp, u = _inputs(rng, B, V, dtype)
        ws = torch.zeros(_lib.workspace_size(B, V, K, code), dtype=torch.uint8, device="cuda:0")
        for stages in (3, 0):
            want = _call(False, t, code, B, V, T, k, p, mp, tlp, u, K, stages, ws)
            got = _call(True, t, code, B, V, T, k, p, mp, tlp, u, K, stages)
            for a, b in zip(want, got):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (dtype, B, V, stages)


def test_noalloc_refuses_oversized_shapes():
    B, V = 4096, 262144
    assert _lib.workspace_size(B, V, 0, _lib.DTYPE_BF16) > _lib.NOALLOC_SCRATCH_BYTES
    err = P()
    rc = _lib.load().mlxf_sample_noalloc(P(16), _lib.DTYPE_BF16, B, V, V, None, None, None, None, None,
                                         None, P(16), None, None, None, 0, 0, None, ctypes.byref(err))
    assert rc == _lib.EWORKSPACE
    msg = ctypes.string_at(err.value).decode()
    _lib.load().mlxf_string_free(err)
    assert "scratch" in msg
