"""Host-side mirror of mlxforge's sampler interface over the HIP C ABI.

* ``SamplingParams`` / ``SampleResult`` mirror src/sample/sampler.h:15-45.
* ``sample_rows`` is the decode-step boundary: what Worker::sample_rows +
  finalize_sample (src/runtime/worker.cpp:448-514) compute, as one launch
  sequence over all rows with per-row parameter arrays.
* ``Sampler.sample`` / ``Sampler.greedy`` mirror the per-call static API
  (src/sample/sampler.h:51-61) with one parameter set for every row.
* ``apply_penalties`` penalizes the logits in place (the reference's `adj`,
  src/sample/sampler.cpp:122-144) before they are sampled.

PyTorch provides device memory and the current stream only; every result is
computed by libmlxf_sampler.so.  The MLX PRNG key of the reference is replaced
by one caller-supplied uniform per row (the inverse-CDF draw of the C ABI).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16,
           torch.float16: _lib.DTYPE_F16}


@dataclass
class SamplingParams:
    """Per-request knobs with the reference's sentinels (src/sample/sampler.h:15-36)."""
    temperature: float = 1.0   # <= 0 => greedy
    top_k: int = 0             # <= 0 => disabled
    top_p: float = 1.0         # >= 1 => disabled
    min_p: float = 0.0         # <= 0 => disabled; applied after top-p
    repetition_penalty: float = 1.0
    frequency_penalty: float = 0.0
    presence_penalty: float = 0.0
    seed: int = 0
    top_logprobs: int = -1     # -1 off, 0 chosen only, N > 0 alternatives

    def has_penalties(self) -> bool:
        return (self.repetition_penalty != 1.0 or self.frequency_penalty != 0.0
                or self.presence_penalty != 0.0)


@dataclass
class SampleResult:
    """src/sample/sampler.h:38-45 (logprobs are fp32 for every input dtype)."""
    tokens: torch.Tensor         # (B,) int32
    logprobs: torch.Tensor       # (B,) fp32
    top_tokens: torch.Tensor     # (B, K) int32
    top_logprobs: torch.Tensor   # (B, K) fp32


class Workspace:
    """Caller-owned device scratch, grown on demand and reused across steps."""

    def __init__(self, device=None):
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.buf = None

    def get(self, B: int, V: int, K_max: int, dtype: int) -> torch.Tensor:
        need = _lib.workspace_size(B, V, K_max, dtype)
        if self.buf is None or self.buf.numel() < need:
            # Zero-filled once (the per-row counters start at 0; every call leaves
            # them at 0).  torch's caching allocator returns >= 512-byte aligned blocks.
            self.buf = torch.zeros(max(need, 256), dtype=torch.uint8, device=self.device)
        return self.buf


_default_ws: dict = {}


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _param(x, B, dtype, device):
    if x is None:
        return None
    if not torch.is_tensor(x):
        if isinstance(x, (int, float)):
            return torch.full((B,), x, dtype=dtype, device=device)
        x = torch.as_tensor(x, dtype=dtype).reshape(-1).to(device)
    if x.dtype != dtype or x.device != device or not x.is_contiguous() or x.numel() != B:
        raise ValueError(f"per-row parameter must be a contiguous {dtype} tensor of {B} on {device}")
    return x


def _host_view(x, B):
    """Host copy of a per-row parameter given as a scalar / sequence / numpy
    array; None when it is a device tensor (then the host does not know it)."""
    import numpy as np
    if x is None:
        return "off"
    if torch.is_tensor(x):
        return None
    return np.broadcast_to(np.asarray(x), (B,))


def sample_rows(logits: torch.Tensor, temperature=None, top_k=None, top_p=None,
                top_logprobs=None, uniforms=None, K_max: int = 0, V: int | None = None,
                workspace: Workspace | None = None, refine_stages: int | None = None,
                min_p=None) -> SampleResult:
    """Sample one token per row of a [B, row_stride] logits view.

    Per-row parameters are device tensors of length B (or Python scalars /
    host sequences, which are copied); None disables the knob (temperature
    None = all greedy; min_p None = off).  refine_stages: refine stages to launch (0..3); by
    default derived from the parameters when they are all known on the host
    (mlxf_sampler_refine_stages: 0, 1 or 2), else 2 (mlxf_sample's count).
    """
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be a [B, V] view with unit stride along V")
    if logits.dtype not in _DTYPES:
        raise ValueError(f"unsupported logits dtype {logits.dtype}")
    dev = logits.device
    B = logits.shape[0]
    V = logits.shape[1] if V is None else V
    code = _DTYPES[logits.dtype]
    if refine_stages is None:
        hv = [_host_view(x, B) for x in (temperature, top_k, top_p)]
        if any(h is None for h in hv):
            refine_stages = 2
        else:
            hv = [None if isinstance(h, str) else h for h in hv]
            refine_stages = _lib.refine_stages(B, V, code, *hv)
    T = _param(temperature, B, torch.float32, dev)
    k = _param(top_k, B, torch.int32, dev)
    p = _param(top_p, B, torch.float32, dev)
    mp = _param(min_p, B, torch.float32, dev)
    tlp = _param(top_logprobs, B, torch.int32, dev)
    u = _param(uniforms, B, torch.float32, dev)
    ids = torch.empty(B, dtype=torch.int32, device=dev)
    lp = torch.empty(B, dtype=torch.float32, device=dev)
    top_ids = torch.empty((B, K_max), dtype=torch.int32, device=dev)
    top_lp = torch.empty((B, K_max), dtype=torch.float32, device=dev)
    if workspace is None:
        workspace = _default_ws.setdefault(dev, Workspace(dev))
    ws = workspace.get(B, V, K_max, code)
    stream = torch.cuda.current_stream(dev).cuda_stream
    err = ctypes.c_void_p()
    rc = _lib.load().mlxf_sample_ex(
        _ptr(logits), code, B, V, logits.stride(0), _ptr(T), _ptr(k), _ptr(p), _ptr(mp), _ptr(tlp),
        _ptr(u),
        _ptr(ids), _ptr(lp), _ptr(top_ids) if K_max else None, _ptr(top_lp) if K_max else None,
        K_max, _ptr(ws), ws.numel(), int(refine_stages), ctypes.c_void_p(stream), ctypes.byref(err))
    _lib.check(rc, err)
    return SampleResult(ids, lp, top_ids, top_lp)


class PenaltyWorkspace:
    """Caller-owned counter array of mlxf_apply_penalties (zeroed once, left zero)."""

    def __init__(self, device=None):
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.buf = None

    def get(self, B: int, V: int) -> torch.Tensor:
        n = ctypes.c_size_t()
        err = ctypes.c_void_p()
        _lib.check(_lib.load().mlxf_penalties_workspace_size(B, V, ctypes.byref(n), ctypes.byref(err)), err)
        if self.buf is None or self.buf.numel() < n.value:
            self.buf = torch.zeros(n.value, dtype=torch.uint8, device=self.device)
        return self.buf


_default_pen_ws: dict = {}


def apply_penalties(logits: torch.Tensor, history: torch.Tensor, hist_len=None, repetition=None,
                    frequency=None, presence=None, V: int | None = None,
                    workspace: PenaltyWorkspace | None = None) -> torch.Tensor:
    """Repetition / frequency / presence penalties on a [B, row_stride] logits
    view, in place (src/sample/sampler.cpp:95-133): the `adj` the sampler then
    reads.  history: [B, N] int32 device tensor; hist_len: per-row used length
    (None: N).  Per-row knobs as in sample_rows (None: off).  Returns logits."""
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be a [B, V] view with unit stride along V")
    if history.dim() != 2 or history.dtype != torch.int32 or history.stride(1) != 1:
        raise ValueError("history must be a [B, N] int32 tensor with unit stride along N")
    dev = logits.device
    B = logits.shape[0]
    V = logits.shape[1] if V is None else V
    code = _DTYPES[logits.dtype]
    hl = _param(hist_len, B, torch.int32, dev)
    rep = _param(repetition, B, torch.float32, dev)
    fq = _param(frequency, B, torch.float32, dev)
    ps = _param(presence, B, torch.float32, dev)
    if workspace is None:
        workspace = _default_pen_ws.setdefault(dev, PenaltyWorkspace(dev))
    ws = workspace.get(B, V)
    stream = torch.cuda.current_stream(dev).cuda_stream
    err = ctypes.c_void_p()
    rc = _lib.load().mlxf_apply_penalties(
        _ptr(logits), code, B, V, logits.stride(0), _ptr(history), history.stride(0), _ptr(hl),
        _ptr(rep), _ptr(fq), _ptr(ps), _ptr(ws), ws.numel(), ctypes.c_void_p(stream), ctypes.byref(err))
    _lib.check(rc, err)
    return logits


def uniforms(seed: torch.Tensor, step, out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-row draw uniforms from (seed, step) on the device (Philox4x32-10,
    mlxf_uniforms): the replacement of the reference's per-row MLX key split
    each step (src/runtime/worker.cpp:416,465-466).  seed: (B,) int64 device
    tensor (bit pattern of the uint64 seed); step: int (same for every row) or
    a (B,) int64 device tensor."""
    if seed.dim() != 1 or seed.dtype != torch.int64 or not seed.is_contiguous():
        raise ValueError("seed must be a contiguous (B,) int64 tensor")
    dev = seed.device
    B = seed.shape[0]
    if out is None:
        out = torch.empty(B, dtype=torch.float32, device=dev)
    st_t = step if torch.is_tensor(step) else None
    if st_t is not None and (st_t.dtype != torch.int64 or st_t.numel() != B or not st_t.is_contiguous()):
        raise ValueError("step must be an int or a contiguous (B,) int64 tensor")
    stream = torch.cuda.current_stream(dev).cuda_stream
    err = ctypes.c_void_p()
    rc = _lib.load().mlxf_uniforms(B, _ptr(seed), _ptr(st_t) if st_t is not None else None,
                                   0 if st_t is not None else int(step) & (2**64 - 1),
                                   _ptr(out), ctypes.c_void_p(stream), ctypes.byref(err))
    _lib.check(rc, err)
    return out


def apply_mask(logits: torch.Tensor, allowed_bits: torch.Tensor, V: int | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """Grammar-constrained rows (src/runtime/worker.cpp:455-459): an fp32
    [B, V] copy with -inf where the bit mask (int32 [B, ceil(V/32)], bit 1 =
    allowed) forbids a token; rows with no allowed token are left unmasked.
    Sample the result as fp32 logits, as the reference samples the promoted
    row."""
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be a [B, V] view with unit stride along V")
    if allowed_bits.dim() != 2 or allowed_bits.dtype != torch.int32 or allowed_bits.stride(1) != 1:
        raise ValueError("allowed_bits must be a [B, W] int32 tensor with unit stride along W")
    dev = logits.device
    B = logits.shape[0]
    V = logits.shape[1] if V is None else V
    if out is None:
        out = torch.empty((B, V), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    err = ctypes.c_void_p()
    rc = _lib.load().mlxf_apply_mask(_ptr(logits), _DTYPES[logits.dtype], B, V, logits.stride(0),
                                     _ptr(allowed_bits), allowed_bits.stride(0), _ptr(out), out.stride(0),
                                     ctypes.c_void_p(stream), ctypes.byref(err))
    _lib.check(rc, err)
    return out


class FilterWorkspace:
    """Caller-owned scratch of the filter calls (no initialisation needed)."""

    def __init__(self, device=None):
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.buf = None

    def get(self, B: int, V: int) -> torch.Tensor:
        need = _lib.filter_workspace_size(B, V)
        if self.buf is None or self.buf.numel() < need:
            # torch's caching allocator returns >= 512-byte aligned blocks
            self.buf = torch.empty(max(need, 256), dtype=torch.uint8, device=self.device)
        return self.buf


_default_filter_ws: dict = {}


def _filter_out(logits: torch.Tensor, V, out, workspace=None):
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be a [B, V] view with unit stride along V")
    if logits.dtype not in _DTYPES:
        raise ValueError(f"unsupported logits dtype {logits.dtype}")
    B = logits.shape[0]
    V = logits.shape[1] if V is None else V
    if out is None:
        out = torch.empty((B, V), dtype=logits.dtype, device=logits.device)
    elif out.dtype != logits.dtype or out.dim() != 2 or out.stride(1) != 1:
        raise ValueError("out must be a [B, V] view of the logits' dtype with unit stride along V")
    if workspace is None:
        workspace = _default_filter_ws.setdefault(logits.device, FilterWorkspace(logits.device))
    ws = workspace.get(B, V)
    stream = ctypes.c_void_p(torch.cuda.current_stream(logits.device).cuda_stream)
    return B, V, out, (_ptr(ws), ws.numel()), stream


def filter_logits(logits: torch.Tensor, temperature=None, top_k=None, top_p=None, min_p=None,
                  V: int | None = None, out: torch.Tensor | None = None,
                  workspace: FilterWorkspace | None = None) -> torch.Tensor:
    """z' = logits / temperature (rounded to the logits dtype) with the
    entries that top-k, top-p and min_p remove set to -inf, per row, as
    Sampler::sample filters before its draw (src/sample/sampler.cpp:158-163).
    Per-row parameters as in sample_rows; None = that step off.  out may be
    logits itself (in place)."""
    B, V, out, ws, stream = _filter_out(logits, V, out, workspace)
    dev = logits.device
    T = _param(temperature, B, torch.float32, dev)
    k = _param(top_k, B, torch.int32, dev)
    p = _param(top_p, B, torch.float32, dev)
    mp = _param(min_p, B, torch.float32, dev)
    err = ctypes.c_void_p()
    rc = _lib.load().mlxf_filter_logits(_ptr(logits), _DTYPES[logits.dtype], B, V, logits.stride(0), _ptr(T),
                                        _ptr(k), _ptr(p), _ptr(mp), _ptr(out), out.stride(0), *ws, stream,
                                        ctypes.byref(err))
    _lib.check(rc, err)
    return out


def apply_top_k(logits: torch.Tensor, k: int, out: torch.Tensor | None = None,
                workspace: FilterWorkspace | None = None) -> torch.Tensor:
    """Sampler::apply_top_k (src/sample/sampler.cpp:63-68): entries below the
    k-th largest (counting multiplicity) set to -inf."""
    B, V, out, ws, stream = _filter_out(logits, None, out, workspace)
    err = ctypes.c_void_p()
    rc = _lib.load().mlxf_apply_top_k(_ptr(logits), _DTYPES[logits.dtype], B, V, logits.stride(0), int(k),
                                      _ptr(out), out.stride(0), *ws, stream, ctypes.byref(err))
    _lib.check(rc, err)
    return out


def apply_top_p(logits: torch.Tensor, p: float, out: torch.Tensor | None = None,
                workspace: FilterWorkspace | None = None) -> torch.Tensor:
    """Sampler::apply_top_p (src/sample/sampler.cpp:70-85): entries past the
    smallest (value desc, index asc) prefix whose mass reaches p set to -inf."""
    B, V, out, ws, stream = _filter_out(logits, None, out, workspace)
    err = ctypes.c_void_p()
    rc = _lib.load().mlxf_apply_top_p(_ptr(logits), _DTYPES[logits.dtype], B, V, logits.stride(0), float(p),
                                      _ptr(out), out.stride(0), *ws, stream, ctypes.byref(err))
    _lib.check(rc, err)
    return out


def apply_min_p(logits: torch.Tensor, min_p: float, out: torch.Tensor | None = None,
                workspace: FilterWorkspace | None = None) -> torch.Tensor:
    """Sampler::apply_min_p (src/sample/sampler.cpp:87-93): entries whose
    probability is below min_p times the largest set to -inf."""
    B, V, out, ws, stream = _filter_out(logits, None, out, workspace)
    err = ctypes.c_void_p()
    rc = _lib.load().mlxf_apply_min_p(_ptr(logits), _DTYPES[logits.dtype], B, V, logits.stride(0),
                                      float(min_p), _ptr(out), out.stride(0), *ws, stream, ctypes.byref(err))
    _lib.check(rc, err)
    return out


def greedy(logits: torch.Tensor, workspace: Workspace | None = None) -> torch.Tensor:
    """argmax per row, lowest index on ties (src/sample/sampler.cpp:59-61)."""
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be a [B, V] view with unit stride along V")
    dev = logits.device
    B, V = logits.shape
    code = _DTYPES[logits.dtype]
    ids = torch.empty(B, dtype=torch.int32, device=dev)
    if workspace is None:
        workspace = _default_ws.setdefault(dev, Workspace(dev))
    ws = workspace.get(B, V, 0, code)
    stream = torch.cuda.current_stream(dev).cuda_stream
    err = ctypes.c_void_p()
    rc = _lib.load().mlxf_greedy(_ptr(logits), code, B, V, logits.stride(0), _ptr(ids), _ptr(ws),
                                 ws.numel(), ctypes.c_void_p(stream), ctypes.byref(err))
    _lib.check(rc, err)
    return ids


class Sampler:
    """Per-call API of src/sample/sampler.h:47-79, one parameter set for all rows."""

    @staticmethod
    def sample(logits: torch.Tensor, params: SamplingParams, uniforms, history=None) -> SampleResult:
        """history: [B, N] int32 device tensor; with penalties in params the
        logits are penalized in place first (src/sample/sampler.cpp:144)."""
        if params.has_penalties() and history is not None and history.shape[1] > 0:
            apply_penalties(logits, history, repetition=params.repetition_penalty,
                            frequency=params.frequency_penalty, presence=params.presence_penalty)
        B, V = logits.shape
        K = min(max(params.top_logprobs, 0), V)
        # Sampler::sample always returns the chosen-token logprob (sampler.cpp:151-154).
        res = sample_rows(logits, temperature=params.temperature, top_k=params.top_k,
                          top_p=params.top_p, top_logprobs=max(params.top_logprobs, 0),
                          uniforms=uniforms, K_max=K, min_p=params.min_p)
        return res

    @staticmethod
    def greedy(logits: torch.Tensor) -> torch.Tensor:
        return greedy(logits)

    @staticmethod
    def apply_top_k(logits: torch.Tensor, k: int) -> torch.Tensor:
        return apply_top_k(logits, k)

    @staticmethod
    def apply_top_p(logits: torch.Tensor, p: float) -> torch.Tensor:
        return apply_top_p(logits, p)

    @staticmethod
    def apply_min_p(logits: torch.Tensor, min_p: float) -> torch.Tensor:
        return apply_min_p(logits, min_p)
