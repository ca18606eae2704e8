"""ctypes binding of the CPU oracle (oracle/sampler_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
bench.py's cpu_baseline leg, always as the checker.  The product package
(mlxforge_amd) never imports this module.

Arguments mirror the product's C ABI ``mlxf_sample`` (include/mlxf_sampler.h)
with host numpy arrays in place of device pointers.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, BF16, F16 = 0, 1, 2
FLAG_GREEDY, FLAG_TOPP_AMBIG, FLAG_DRAW_AMBIG, FLAG_MINP_AMBIG = 1, 2, 4, 8

_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE] + (["-B"] if force else []), check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = _configure(ctypes.CDLL(LIB_PATH))
    return _lib


def native_lib(out_dir: str):
    """The CPU baseline's build of the same source (-O3 -march=native), compiled
    on the machine that times it into out_dir (make -C oracle native)."""
    subprocess.run(["make", "-s", "-C", HERE, "native", f"OUT={out_dir}"], check=True)
    return _configure(ctypes.CDLL(os.path.join(out_dir, "liboracle_native.so")))


def _configure(L):
    """Argument and result types of every exported function."""
    P = ctypes.c_void_p
    L.orc_sample.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_long,
                             P, P, P, P, P, P, P, P, P, ctypes.c_int, P, P, ctypes.c_int]
    L.orc_sample.restype = ctypes.c_int
    L.orc_sample_ex.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_long,
                                P, P, P, P, P, P, P, P, P, P, ctypes.c_int, P, P, ctypes.c_int]
    L.orc_sample_ex.restype = ctypes.c_int
    L.orc_filter_row.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                 ctypes.c_int, ctypes.c_float, ctypes.c_float, P]
    L.orc_filter_row.restype = ctypes.c_int
    L.orc_round_bf16.argtypes = [ctypes.c_float]
    L.orc_round_bf16.restype = ctypes.c_float
    L.orc_round_f16.argtypes = [ctypes.c_float]
    L.orc_round_f16.restype = ctypes.c_float
    L.orc_greedy_row.argtypes = [P, ctypes.c_int]
    L.orc_greedy_row.restype = ctypes.c_int
    L.orc_lse_row.argtypes = [P, ctypes.c_int]
    L.orc_lse_row.restype = ctypes.c_double
    L.orc_draw_row.argtypes = [P, ctypes.c_int, ctypes.c_float, P]
    L.orc_draw_row.restype = ctypes.c_int
    L.orc_apply_penalties.argtypes = [P, ctypes.c_int, ctypes.c_int, P, ctypes.c_int,
                                      ctypes.c_float, ctypes.c_float, ctypes.c_float]
    L.orc_apply_penalties.restype = None
    L.orc_philox4x32_10.argtypes = [P, P, P]
    L.orc_philox4x32_10.restype = None
    L.orc_uniforms.argtypes = [ctypes.c_int, P, P, P]
    L.orc_uniforms.restype = None
    L.orc_admissible.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int,
                                 ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_double,
                                 P, ctypes.c_int]
    L.orc_admissible.restype = ctypes.c_int
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def dtype_code(arr: np.ndarray, dtype: int | None = None) -> int:
    if dtype is not None:
        return dtype
    if arr.dtype == np.float32:
        return F32
    if arr.dtype == np.float16:
        return F16
    raise ValueError("pass dtype=BF16 explicitly for uint16 bf16 bit patterns")


def sample(logits: np.ndarray, T=None, k=None, p=None, tlp=None, u=None, K_max: int = 0,
           dtype: int | None = None, V: int | None = None, nthreads: int | None = None,
           min_p=None, L=None):
    """Run the oracle over a [B, row_stride] host array.

    For bf16, pass the raw uint16 bit patterns with dtype=BF16.  L: a library
    from native_lib() instead of the default build.
    Returns dict(ids, lp, top_ids, top_lp, flags, margins).
    """
    logits = np.ascontiguousarray(logits)
    B, stride = logits.shape
    V = stride if V is None else V
    code = dtype_code(logits, dtype)
    f = lambda a, t: None if a is None else np.ascontiguousarray(np.asarray(a, dtype=t).reshape(B))
    T, p, u, mp = f(T, np.float32), f(p, np.float32), f(u, np.float32), f(min_p, np.float32)
    k, tlp = f(k, np.int32), f(tlp, np.int32)
    ids = np.zeros(B, np.int32)
    lp = np.zeros(B, np.float32)
    top_ids = np.zeros((B, max(K_max, 1)), np.int32)
    top_lp = np.zeros((B, max(K_max, 1)), np.float32)
    flags = np.zeros(B, np.int32)
    margins = np.zeros((B, 2), np.float64)
    if nthreads is None:
        nthreads = min(os.cpu_count() or 1, 16)
    rc = (L or lib()).orc_sample_ex(_ptr(logits), code, B, V, stride, _ptr(T), _ptr(k), _ptr(p), _ptr(mp),
                             _ptr(tlp), _ptr(u), _ptr(ids), _ptr(lp), _ptr(top_ids), _ptr(top_lp),
                             K_max, _ptr(flags), _ptr(margins), nthreads)
    if rc != 0:
        raise ValueError("orc_sample rejected its arguments")
    return dict(ids=ids, lp=lp, top_ids=top_ids[:, :K_max], top_lp=top_lp[:, :K_max],
                flags=flags, margins=margins)


AMBIG_EPS = 1e-6
AMBIG = FLAG_TOPP_AMBIG | FLAG_DRAW_AMBIG | FLAG_MINP_AMBIG


def admissible(row: np.ndarray, dtype: int, T=0.0, k=0, p=1.0, min_p=0.0, u=0.0,
               eps: float = AMBIG_EPS, cap: int = 4096):
    """Every id one row can produce when p, u and min_p each move by up to eps
    (the checker of rows the ambiguity rule excludes from the bit-exact
    comparison).  row: the row's host elements (float32, float16, or bf16 bit
    patterns with dtype=BF16).  Returns a sorted list, or None when the row has
    more variants than cap."""
    row = np.ascontiguousarray(row)
    out = np.zeros(cap, np.int32)
    n = lib().orc_admissible(_ptr(row), dtype, row.size, float(T), int(k), float(p), float(min_p),
                             float(u), eps, _ptr(out), cap)
    if n == -2:
        raise ValueError("orc_admissible rejected its arguments")
    return None if n < 0 else sorted(out[:n].tolist())


def check_rows(ids, ref: dict, logits: np.ndarray, dtype: int, T=None, k=None, p=None, min_p=None,
               u=None, V: int | None = None) -> dict:
    """Ids of one call (ids) against an oracle result (ref, from sample() on the
    same inputs): every row must be the oracle's id, or -- for a row the oracle
    flags as ambiguous -- one of its admissible ids.  Returns the counts
    rows / excluded (flagged) / excluded_matching (flagged, same id as the
    oracle) / excluded_admissible (flagged, an admissible id) and the rows that
    fail ("bad": neither)."""
    ids = np.asarray(ids)
    B = ids.shape[0]
    V = logits.shape[1] if V is None else V
    g = lambda a, d: d if a is None else a[r]
    amb = (ref["flags"] & AMBIG) != 0
    same = ids == ref["ids"]
    bad, adm_ok = [], 0
    for r in range(B):
        if same[r]:
            if amb[r]:
                adm_ok += 1
            continue
        if not amb[r]:
            bad.append(r)
            continue
        a = admissible(logits[r, :V], dtype, T=g(T, 0.0), k=g(k, 0), p=g(p, 1.0), min_p=g(min_p, 0.0),
                       u=g(u, 0.0))
        if a is not None and int(ids[r]) in a:
            adm_ok += 1
        else:
            bad.append(r)
    return dict(rows=int(B), excluded=int(amb.sum()), excluded_matching=int((amb & same).sum()),
                excluded_admissible=int(adm_ok), bad=bad)


def filter_row(z, T=0.0, k=0, p=1.0, min_p=0.0, dtype: int = F32, with_flags: bool = False):
    """z' after temperature / top-k / top-p / min-p (dropped entries are -inf);
    with_flags: (z', ambiguity flags of the top-p and min_p cutoffs)."""
    z = np.ascontiguousarray(np.asarray(z, np.float32))
    out = np.zeros_like(z)
    rc = lib().orc_filter_row(_ptr(z), z.size, dtype, T, k, p, min_p, _ptr(out))
    assert rc >= 0
    return (out, rc) if with_flags else out


def apply_penalties(z, hist, rep=1.0, freq=0.0, pres=0.0, dtype: int = F32) -> np.ndarray:
    """Penalized copy of one row (float32 values of the logits dtype)."""
    z = np.array(z, np.float32)
    h = np.ascontiguousarray(np.asarray(hist, np.int32))
    lib().orc_apply_penalties(_ptr(z), z.size, dtype, _ptr(h), h.size, rep, freq, pres)
    return z


def philox4x32_10(ctr, key) -> list:
    c = np.ascontiguousarray(np.asarray(ctr, np.uint32))
    k = np.ascontiguousarray(np.asarray(key, np.uint32))
    o = np.zeros(4, np.uint32)
    lib().orc_philox4x32_10(_ptr(c), _ptr(k), _ptr(o))
    return [int(x) for x in o]


def uniforms(seed, step) -> np.ndarray:
    seed = np.ascontiguousarray(np.asarray(seed, np.uint64))
    step = np.ascontiguousarray(np.broadcast_to(np.asarray(step, np.uint64), seed.shape))
    u = np.zeros(seed.size, np.float32)
    lib().orc_uniforms(seed.size, _ptr(seed), _ptr(step), _ptr(u))
    return u


def apply_mask(z, allowed) -> np.ndarray:
    """row + the grammar's additive fp32 mask (0 allowed, -inf not), as MLX
    evaluates it: an fp32 row (src/runtime/worker.cpp:455-459).  A row with no
    allowed token gets the zero mask (:175-177).  z: float32 values of the
    logits dtype; allowed: bool per token."""
    z = np.asarray(z, np.float32)
    allowed = np.asarray(allowed, bool)
    if not allowed.any():
        allowed = np.ones_like(allowed)
    mask = np.where(allowed, np.float32(0.0), np.float32(-np.inf)).astype(np.float32)
    return (z + mask).astype(np.float32)


def pack_bits(allowed) -> np.ndarray:
    """bool [B, V] -> uint32 [B, ceil(V / 32)], bit (i & 31) of word i >> 5."""
    allowed = np.asarray(allowed, bool)
    B, V = allowed.shape
    W = (V + 31) // 32
    padded = np.zeros((B, W * 32), bool)
    padded[:, :V] = allowed
    bits = padded.reshape(B, W, 32).astype(np.uint64) << np.arange(32, dtype=np.uint64)
    return bits.sum(axis=2).astype(np.uint32)


def greedy_row(z) -> int:
    z = np.ascontiguousarray(np.asarray(z, np.float32))
    return lib().orc_greedy_row(_ptr(z), z.size)


def lse_row(z) -> float:
    z = np.ascontiguousarray(np.asarray(z, np.float32))
    return lib().orc_lse_row(_ptr(z), z.size)


def draw_row(zs, u: float):
    zs = np.ascontiguousarray(np.asarray(zs, np.float32))
    m = np.zeros(1, np.float64)
    i = lib().orc_draw_row(_ptr(zs), zs.size, u, _ptr(m))
    return i, float(m[0])


def round_bf16(x: float) -> float:
    return lib().orc_round_bf16(x)


def round_f16(x: float) -> float:
    return lib().orc_round_f16(x)
