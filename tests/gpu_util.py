"""Helpers shared by the GPU parity tests: run the HIP path through the C ABI
and compare it with the CPU oracle under the north-star rules.

  * token ids bit-exact, except rows the oracle flags as ambiguous (top-p
    cutoff, min_p threshold or draw boundary within 1e-6 of the compared
    quantity); such a row's id must be one of the ids the oracle gives when
    p, u and min_p move by up to 1e-6 (oracle.admissible), and the counts are
    reported;
  * logprobs within 1e-5 (fp32 logits) or 2e-3 (bf16 / fp16 logits);
  * top_logprobs ids bit-exact, values within the same tolerance.
"""
from __future__ import annotations

import numpy as np
import torch

from mlxforge_amd import sampler
from oracle import oracle as orc

DT = {"f32": (torch.float32, orc.F32), "bf16": (torch.bfloat16, orc.BF16),
      "f16": (torch.float16, orc.F16)}
TOL = {"f32": 1e-5, "bf16": 2e-3, "f16": 2e-3}


def host_values(host: np.ndarray, dtype: str) -> np.ndarray:
    """Host logits as float32 values (bf16 given as uint16 bit patterns)."""
    if dtype == "bf16":
        return (np.asarray(host).astype(np.uint32) << np.uint32(16)).view(np.float32)
    return np.asarray(host).astype(np.float32)


def to_device(host: np.ndarray, dtype: str, device="cuda:0") -> torch.Tensor:
    """float32 / float16 arrays as is; bf16 given as uint16 bit patterns."""
    if dtype == "bf16":
        t = torch.from_numpy(host.view(np.int16)).view(torch.bfloat16)
    else:
        t = torch.from_numpy(host)
    return t.to(device)


def gpu_sample(logits_dev, T=None, k=None, p=None, tlp=None, u=None, K_max=0, V=None,
               stages=None, min_p=None):
    """stages: refine stages to launch (None: all three)."""
    dev = logits_dev.device
    f = lambda a, t: None if a is None else torch.as_tensor(np.asarray(a), dtype=t).to(dev)
    res = sampler.sample_rows(logits_dev, temperature=f(T, torch.float32), top_k=f(k, torch.int32),
                              top_p=f(p, torch.float32), top_logprobs=f(tlp, torch.int32),
                              uniforms=f(u, torch.float32), K_max=K_max, V=V,
                              refine_stages=3 if stages is None else stages,
                              min_p=f(min_p, torch.float32))
    torch.cuda.synchronize()
    return dict(ids=res.tokens.cpu().numpy(), lp=res.logprobs.cpu().numpy(),
                top_ids=res.top_tokens.cpu().numpy(), top_lp=res.top_logprobs.cpu().numpy())


def oracle_sample(host, dtype, T=None, k=None, p=None, tlp=None, u=None, K_max=0, V=None,
                  min_p=None):
    o = orc.sample(host, T=T, k=k, p=p, tlp=tlp, u=u, K_max=K_max, dtype=DT[dtype][1], V=V,
                   min_p=min_p)
    arr = lambda a, t: None if a is None else np.asarray(a, t).reshape(-1)
    o["inputs"] = dict(logits=np.asarray(host), dtype=DT[dtype][1], T=arr(T, np.float32),
                       k=arr(k, np.int32), p=arr(p, np.float32), min_p=arr(min_p, np.float32),
                       u=arr(u, np.float32), V=V)
    return o


def compare(g, o, dtype, tlp=None, label=""):
    """Assert parity; returns a small report dict.  Every row is checked: the
    oracle's id, or for a flagged row one of its admissible ids."""
    B = o["ids"].shape[0]
    amb = (o["flags"] & orc.AMBIG) != 0
    same = g["ids"] == o["ids"]
    rep = orc.check_rows(g["ids"], o, **o["inputs"])
    bad = np.asarray(rep["bad"], dtype=np.int64)
    assert bad.size == 0, (f"{label}: {bad.size} rows are neither the oracle's id nor admissible, "
                           f"first rows {bad[:8].tolist()} gpu={g['ids'][bad[:8]].tolist()} "
                           f"oracle={o['ids'][bad[:8]].tolist()} "
                           f"flags={o['flags'][bad[:8]].tolist()} "
                           f"margins={o['margins'][bad[:8]].tolist()}")
    assert rep["excluded_admissible"] == rep["excluded"]
    tol = TOL[dtype]
    tlp = np.full(B, -1) if tlp is None else np.asarray(tlp)
    lp_rows = tlp >= 0
    lp_err = 0.0
    if lp_rows.any():
        # a row whose (admissible) id differs from the oracle's: the expected
        # logprob is its own logit minus the row's LSE, which the oracle's
        # chosen logprob gives
        z = host_values(o["inputs"]["logits"], dtype)
        rows = np.arange(B)
        lse = z[rows, o["ids"]].astype(np.float64) - o["lp"].astype(np.float64)
        want = np.where(same, o["lp"].astype(np.float64), z[rows, g["ids"]].astype(np.float64) - lse)
        a, b = g["lp"][lp_rows].astype(np.float64), want[lp_rows]
        fin = np.isfinite(b)
        assert np.array_equal(np.isfinite(a), fin), f"{label}: logprob finiteness differs"
        if fin.any():
            lp_err = float(np.abs(a[fin] - b[fin]).max())
        assert lp_err <= tol, f"{label}: logprob error {lp_err} > {tol}"
    if o["top_ids"].shape[1] > 0:
        assert np.array_equal(g["top_ids"], o["top_ids"]), f"{label}: top_logprobs ids differ"
        a, b = g["top_lp"].astype(np.float64), o["top_lp"].astype(np.float64)
        fin = np.isfinite(b)
        assert np.array_equal(np.isfinite(a), fin)
        if fin.any():
            e = float(np.abs(a[fin] - b[fin]).max())
            assert e <= tol, f"{label}: top_logprobs error {e} > {tol}"
            lp_err = max(lp_err, e)
    return dict(rows=B, excluded=int(amb.sum()), excluded_matching=int((amb & same).sum()),
                excluded_admissible=rep["excluded_admissible"], lp_max_err=lp_err)
