"""ctypes binding of libmlxf_sampler.so (the C ABI in include/mlxf_sampler.h).

The library is loaded from this package directory only.  There is no fallback:
if the HIP library is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmlxf_sampler.so")

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
OK, EINVAL, EWORKSPACE, EHIP = 0, -1, -2, -3
MAX_TOP_LOGPROBS = 4096
MAX_VOCAB = 524288

# Every function include/*.h declares.
SYMBOLS = (
    "mlxf_sampler_abi_version",
    "mlxf_sampler_workspace_size",
    "mlxf_sample",
    "mlxf_sample_staged",
    "mlxf_sample_ex",
    "mlxf_penalties_workspace_size",
    "mlxf_apply_penalties",
    "mlxf_uniforms",
    "mlxf_apply_mask",
    "mlxf_sampler_refine_stages",
    "mlxf_sampler_first_pass",
    "mlxf_greedy",
    "mlxf_string_free",
    "mlxf_sampler_workspace_init",
    "mlxf_sample_noalloc",
    "mlxf_filter_workspace_size",
    "mlxf_filter_logits",
    "mlxf_apply_top_k",
    "mlxf_apply_top_p",
    "mlxf_apply_min_p",
)
NOALLOC_SCRATCH_BYTES = 64 << 20

_lib = None


class SamplerError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (code {code})")
        self.code = code


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
    L = ctypes.CDLL(LIB_PATH)
    P, I, I64, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    PP = ctypes.POINTER(ctypes.c_void_p)
    L.mlxf_sampler_abi_version.argtypes = []
    L.mlxf_sampler_abi_version.restype = I
    L.mlxf_sampler_workspace_size.argtypes = [I, I, I, I, ctypes.POINTER(SZ), PP]
    L.mlxf_sampler_workspace_size.restype = I
    L.mlxf_sample.argtypes = [P, I, I, I, I64, P, P, P, P, P, P, P, P, P, I, P, SZ, P, PP]
    L.mlxf_sample.restype = I
    L.mlxf_sample_staged.argtypes = [P, I, I, I, I64, P, P, P, P, P, P, P, P, P, I, P, SZ, I, P, PP]
    L.mlxf_sample_staged.restype = I
    L.mlxf_sample_ex.argtypes = [P, I, I, I, I64, P, P, P, P, P, P, P, P, P, P, I, P, SZ, I, P, PP]
    L.mlxf_sample_ex.restype = I
    L.mlxf_penalties_workspace_size.argtypes = [I, I, ctypes.POINTER(SZ), PP]
    L.mlxf_penalties_workspace_size.restype = I
    L.mlxf_apply_penalties.argtypes = [P, I, I, I, I64, P, I64, P, P, P, P, P, SZ, P, PP]
    L.mlxf_apply_penalties.restype = I
    L.mlxf_uniforms.argtypes = [I, P, P, ctypes.c_uint64, P, P, PP]
    L.mlxf_uniforms.restype = I
    L.mlxf_apply_mask.argtypes = [P, I, I, I, I64, P, I64, P, I64, P, PP]
    L.mlxf_apply_mask.restype = I
    L.mlxf_sampler_first_pass.argtypes = [P, I, I, I, I64, P, P, P, P, P, P, P, P, P, I, P, SZ, P, PP]
    L.mlxf_sampler_first_pass.restype = I
    L.mlxf_sampler_refine_stages.argtypes = [I, I, I, P, P, P]
    L.mlxf_sampler_refine_stages.restype = I
    L.mlxf_greedy.argtypes = [P, I, I, I, I64, P, P, SZ, P, PP]
    L.mlxf_greedy.restype = I
    L.mlxf_filter_workspace_size.argtypes = [I, I, ctypes.POINTER(SZ), PP]
    L.mlxf_filter_workspace_size.restype = I
    L.mlxf_filter_logits.argtypes = [P, I, I, I, I64, P, P, P, P, P, I64, P, SZ, P, PP]
    L.mlxf_filter_logits.restype = I
    L.mlxf_apply_top_k.argtypes = [P, I, I, I, I64, I, P, I64, P, SZ, P, PP]
    L.mlxf_apply_top_k.restype = I
    L.mlxf_apply_top_p.argtypes = [P, I, I, I, I64, ctypes.c_float, P, I64, P, SZ, P, PP]
    L.mlxf_apply_top_p.restype = I
    L.mlxf_apply_min_p.argtypes = [P, I, I, I, I64, ctypes.c_float, P, I64, P, SZ, P, PP]
    L.mlxf_apply_min_p.restype = I
    L.mlxf_sample_noalloc.argtypes = [P, I, I, I, I64, P, P, P, P, P, P, P, P, P, P, I, I, P, PP]
    L.mlxf_sample_noalloc.restype = I
    L.mlxf_sampler_workspace_init.argtypes = [P, SZ, P, PP]
    L.mlxf_sampler_workspace_init.restype = I
    L.mlxf_string_free.argtypes = [P]
    L.mlxf_string_free.restype = None
    _lib = L
    return L


def check(rc: int, err: ctypes.c_void_p) -> None:
    """Raise SamplerError for a negative return code, freeing the message."""
    if rc == OK:
        return
    msg = "mlxf: error"
    if err.value:
        msg = ctypes.string_at(err.value).decode("utf-8", "replace")
        load().mlxf_string_free(err)
    raise SamplerError(rc, msg)


def abi_version() -> int:
    return load().mlxf_sampler_abi_version()


def workspace_size(B: int, V: int, K_max: int, dtype: int) -> int:
    n = ctypes.c_size_t(0)
    err = ctypes.c_void_p()
    rc = load().mlxf_sampler_workspace_size(B, V, K_max, dtype, ctypes.byref(n), ctypes.byref(err))
    check(rc, err)
    return n.value


def filter_workspace_size(B: int, V: int) -> int:
    n = ctypes.c_size_t(0)
    err = ctypes.c_void_p()
    rc = load().mlxf_filter_workspace_size(B, V, ctypes.byref(n), ctypes.byref(err))
    check(rc, err)
    return n.value


def refine_stages(B: int, V: int, dtype: int, T=None, k=None, p=None) -> int:
    """Refine stages a call needs, from host arrays of the per-row temperature,
    top_k and top_p (numpy float32 / int32 / float32, or None for the sentinel)."""
    import numpy as np

    def ptr(a, t):
        if a is None:
            return None, None
        a = np.ascontiguousarray(a, dtype=t)
        return a, a.ctypes.data_as(ctypes.c_void_p)

    Ta, Tp = ptr(T, np.float32)
    ka, kp = ptr(k, np.int32)
    pa, pp = ptr(p, np.float32)
    return load().mlxf_sampler_refine_stages(B, V, dtype, Tp, kp, pp)
