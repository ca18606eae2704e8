"""The C-ABI library loads and exports every symbol include/mlxf_sampler.h
declares; host-side argument checks answer without touching a GPU."""
import ctypes
import glob
import os
import re

import pytest

from mlxforge_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mlxf_sampler.h")
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(mlxf_\w+)\s*\(", text))
    return sorted(names)


def test_header_matches_binding_list():
    assert declared_functions() == sorted(_lib.SYMBOLS)


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    for name in declared_functions():
        assert hasattr(L, name), name


def test_abi_version():
    text = open(HEADER).read()
    want = int(re.search(r"#define MLXF_SAMPLER_ABI_VERSION (\d+)", text).group(1))
    assert _lib.abi_version() == want


def test_workspace_size_is_positive_and_monotone():
    a = _lib.workspace_size(8, 151936, 0, _lib.DTYPE_BF16)
    b = _lib.workspace_size(64, 151936, 20, _lib.DTYPE_F32)
    assert 0 < a < b
    # top_logprobs above the 64-entry lists: the wide kernels' states, slice
    # histograms and per-row lists (K_max entries of 8 bytes) come on top
    c64 = _lib.workspace_size(64, 151936, 64, _lib.DTYPE_F32)
    c65 = _lib.workspace_size(64, 151936, 65, _lib.DTYPE_F32)
    c4k = _lib.workspace_size(64, 151936, 4096, _lib.DTYPE_F32)
    assert c64 < c65 < c4k and c4k - c65 >= 64 * (4096 - 65) * 8


@pytest.mark.parametrize("args", [
    (-1, 10, 0, 0), (1, 0, 0, 0), (1, 10, _lib.MAX_TOP_LOGPROBS + 1, 0), (1, 10, 0, 7),
    (1, _lib.MAX_VOCAB + 1, 0, 0)])
def test_workspace_size_rejects_bad_shapes(args):
    with pytest.raises(_lib.SamplerError) as ei:
        _lib.workspace_size(*args)
    assert ei.value.code == _lib.EINVAL and "mlxf" in str(ei.value)


def test_sample_argument_errors_need_no_gpu():
    L = _lib.load()
    err = ctypes.c_void_p()
    fake = ctypes.c_void_p(0x1000)
    # NULL logits
    rc = L.mlxf_sample(None, 0, 1, 10, 10, None, None, None, None, None, fake, None, None, None,
                       0, fake, 1 << 20, None, ctypes.byref(err))
    assert rc == _lib.EINVAL and err.value
    L.mlxf_string_free(err)
    # row_stride < V
    err = ctypes.c_void_p()
    rc = L.mlxf_sample(fake, 0, 1, 10, 9, None, None, None, None, None, fake, None, None, None,
                       0, fake, 1 << 20, None, ctypes.byref(err))
    assert rc == _lib.EINVAL
    L.mlxf_string_free(err)
    # temperature without uniforms
    err = ctypes.c_void_p()
    rc = L.mlxf_sample(fake, 0, 1, 10, 10, fake, None, None, None, None, fake, None, None, None,
                       0, fake, 1 << 20, None, ctypes.byref(err))
    assert rc == _lib.EINVAL
    L.mlxf_string_free(err)
    # workspace too small
    err = ctypes.c_void_p()
    rc = L.mlxf_sample(fake, 0, 1, 10, 10, None, None, None, None, None, fake, None, None, None,
                       0, fake, 16, None, ctypes.byref(err))
    assert rc == _lib.EWORKSPACE
    L.mlxf_string_free(err)
    # B == 0 is a no-op success; a NULL err pointer is allowed
    assert L.mlxf_sample(None, 0, 0, 10, 10, None, None, None, None, None, None, None, None, None,
                         0, None, 0, None, None) == 0


def test_sample_ex_argument_errors_need_no_gpu():
    L = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    # negative stage count
    err = ctypes.c_void_p()
    rc = L.mlxf_sample_ex(fake, 0, 1, 10, 10, None, None, None, None, None, None, fake, None, None,
                          None, 0, fake, 1 << 20, -1, None, ctypes.byref(err))
    assert rc == _lib.EINVAL and err.value
    L.mlxf_string_free(err)
    # min_p without temperature is fine (greedy rows ignore it); NULL logits is not
    err = ctypes.c_void_p()
    rc = L.mlxf_sample_ex(None, 0, 1, 10, 10, None, None, None, fake, None, None, fake, None, None,
                          None, 0, fake, 1 << 20, 3, None, ctypes.byref(err))
    assert rc == _lib.EINVAL
    L.mlxf_string_free(err)
    assert L.mlxf_sample_ex(None, 0, 0, 10, 10, None, None, None, None, None, None, None, None, None,
                            None, 0, None, 0, 0, None, None) == 0


def test_refine_stage_hint_from_host_parameters():
    """Host-side stage count: greedy and top-k <= 63 rows need none, temperature-
    only rows one (the kept-mass pass), anything else two."""
    import numpy as np
    rs = lambda T, k=None, p=None, B=4, V=1000, dt=_lib.DTYPE_F32: _lib.refine_stages(B, V, dt, T, k, p)
    z = np.zeros(4, np.float32)
    assert rs(None) == 0
    assert rs(z) == 0                                            # all greedy
    assert rs(np.full(4, np.nan, np.float32)) == 0               # non-finite T is greedy
    assert rs(np.ones(4, np.float32), np.full(4, 63, np.int32)) == 0
    assert rs(np.ones(4, np.float32), np.full(4, 64, np.int32)) == 2
    assert rs(np.ones(4, np.float32), np.full(4, 5000, np.int32), V=50) == 0  # k clamped to V
    assert rs(np.ones(4, np.float32)) == 1                      # temperature only
    assert rs(np.ones(4, np.float32), None, np.full(4, 1.0, np.float32)) == 1  # p >= 1 is off
    assert rs(np.ones(4, np.float32), None, np.full(4, 0.9, np.float32)) == 2
    assert rs(np.ones(4, np.float32), np.full(4, 20, np.int32), np.full(4, 0.9, np.float32)) == 0
    # bf16: a temperature that rounds to 0 is greedy
    assert rs(np.full(4, 1e-45, np.float32), dt=_lib.DTYPE_BF16) == 0


def test_pre_sampling_entry_points_argument_errors_need_no_gpu():
    L = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    n = ctypes.c_size_t()
    # penalties: workspace size is B * V counters, 256-byte aligned
    assert L.mlxf_penalties_workspace_size(3, 1000, ctypes.byref(n), None) == 0
    assert n.value >= 3 * 1000 * 4 and n.value % 256 == 0
    assert L.mlxf_penalties_workspace_size(-1, 1000, ctypes.byref(n), None) == _lib.EINVAL
    # penalties: bad dtype / shape, missing history, small workspace; nothing to do is a success
    err = ctypes.c_void_p()
    assert L.mlxf_apply_penalties(fake, 9, 1, 10, 10, fake, 4, None, fake, None, None, fake, 1 << 20,
                                  None, ctypes.byref(err)) == _lib.EINVAL
    L.mlxf_string_free(err)
    err = ctypes.c_void_p()
    assert L.mlxf_apply_penalties(fake, 0, 1, 10, 9, fake, 4, None, fake, None, None, fake, 1 << 20,
                                  None, ctypes.byref(err)) == _lib.EINVAL
    L.mlxf_string_free(err)
    err = ctypes.c_void_p()
    assert L.mlxf_apply_penalties(fake, 0, 1, 10, 10, None, 4, None, fake, None, None, fake, 1 << 20,
                                  None, ctypes.byref(err)) == _lib.EINVAL
    L.mlxf_string_free(err)
    err = ctypes.c_void_p()
    assert L.mlxf_apply_penalties(fake, 0, 2, 10, 10, fake, 4, None, fake, None, None, fake, 16,
                                  None, ctypes.byref(err)) == _lib.EWORKSPACE
    L.mlxf_string_free(err)
    assert L.mlxf_apply_penalties(fake, 0, 2, 10, 10, fake, 4, None, None, None, None, None, 0,
                                  None, None) == 0  # no penalty array: nothing to do
    assert L.mlxf_apply_penalties(fake, 0, 2, 10, 10, fake, 0, None, fake, None, None, None, 0,
                                  None, None) == 0  # empty history
    # filters: workspace size grows with B; a missing or small workspace and a
    # misaligned one are refused before any GPU work
    a, b = ctypes.c_size_t(), ctypes.c_size_t()
    assert L.mlxf_filter_workspace_size(8, 151936, ctypes.byref(a), None) == 0
    assert L.mlxf_filter_workspace_size(64, 151936, ctypes.byref(b), None) == 0
    assert 0 < a.value <= b.value and a.value % 256 == 0
    assert L.mlxf_filter_workspace_size(0, 10, ctypes.byref(a), None) == 0 and a.value == 0
    assert L.mlxf_filter_workspace_size(4, 0, ctypes.byref(a), None) == _lib.EINVAL
    out = ctypes.c_void_p(0x100000)
    for ws, nbytes, code in ((None, 1 << 20, _lib.EWORKSPACE), (fake, 16, _lib.EWORKSPACE),
                             (ctypes.c_void_p(0x1008), 1 << 24, _lib.EINVAL)):
        err = ctypes.c_void_p()
        assert L.mlxf_apply_top_k(fake, 0, 2, 10, 10, 3, out, 10, ws, nbytes, None, ctypes.byref(err)) == code
        assert err.value
        L.mlxf_string_free(err)
    # uniforms
    err = ctypes.c_void_p()
    assert L.mlxf_uniforms(-1, fake, None, 0, fake, None, ctypes.byref(err)) == _lib.EINVAL
    L.mlxf_string_free(err)
    err = ctypes.c_void_p()
    assert L.mlxf_uniforms(4, None, None, 0, fake, None, ctypes.byref(err)) == _lib.EINVAL
    L.mlxf_string_free(err)
    assert L.mlxf_uniforms(0, None, None, 0, None, None, None) == 0
    # mask: bad dtype, bits_stride too small, missing output
    for args in ((fake, 7, 1, 100, 100, fake, 4, fake, 100), (fake, 0, 1, 100, 100, fake, 3, fake, 100),
                 (fake, 0, 1, 100, 100, fake, 4, None, 100), (fake, 0, 1, 100, 100, fake, 4, fake, 99)):
        err = ctypes.c_void_p()
        assert L.mlxf_apply_mask(*args, None, ctypes.byref(err)) == _lib.EINVAL and err.value
        L.mlxf_string_free(err)
    assert L.mlxf_apply_mask(None, 0, 0, 100, 100, None, 4, None, 100, None, None) == 0
