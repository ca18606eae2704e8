#!/usr/bin/env python3
"""Benchmark of the MI355X batched token sampler (one decode step = one
mlxf_sample_staged call over a [B, V] logits matrix already resident in HBM).

Default workload: config C3 (B=32, V=151936, fp32, T=1, top-k 50, top-p 0.95),
the configuration the headline metric is quoted on.  Prints ONE JSON line.

Timing: hipEvents (torch.cuda.Event on the stream the library launches on)
around K back-to-back steps after W warm-up steps; the input is rotated over
enough copies to exceed 512 MB so neither L2 nor the 256 MB MALL holds it when
a step starts ("cold" HBM).  A step launches the stage count the host-side
parameters call for (mlxf_sampler_refine_stages); the generic call (plain
mlxf_sample, two refine stages) and all three stages are timed too.  The roofline figure is for the step's
dominant kernel, k_scan1 (the one HBM read of the logits), timed alone through
mlxf_sampler_first_pass.  cpu_baseline times the CPU restatement of the
reference sampler (oracle/, "port") on the same workload with a bounded number
of repetitions.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = ("µs/decode-step and sampled rows/sec at B=32,V=151936; achieved HBM GB/s")
HBM_PEAK_GBPS = 8000.0
ROTATE_BYTES = 512 << 20

# HBM bytes per k_scan1 launch from rocprofv3 FETCH_SIZE and WRITE_SIZE runs
# (separate passes), each scaled by what the counter reads for a plain device
# copy of known size (--copy-calibration): profiles/k_scan1_C3_hbm_traffic.md.
# A counter run cannot share the timed process, so the figure is carried here.
MEASURED_TRAFFIC_BYTES = {3: 20069987}
COPY_CALIBRATION_BYTES = 256 << 20


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Step:
    """Pre-allocated device state for one workload; run() issues one mlxf_sample."""

    def __init__(self, wl, torch, lib, rotate=True, hinted=True):
        import numpy as np
        self.wl, self.torch, self.lib = wl, torch, lib
        dev = torch.device("cuda:0")
        host = wl.logits
        nbytes = host.nbytes
        self.R = max(3, -(-ROTATE_BYTES // nbytes) + 1) if rotate else 1
        t = torch.from_numpy(host.view(np.int16)).view(torch.bfloat16) if wl.dtype == "bf16" \
            else torch.from_numpy(host)
        one = t.to(dev)
        self.buf = one.unsqueeze(0).repeat(self.R, 1, 1).contiguous()
        del one
        d = lambda a, ty: torch.as_tensor(a, dtype=ty).to(dev)
        self.T, self.k, self.p = d(wl.T, torch.float32), d(wl.k, torch.int32), d(wl.p, torch.float32)
        self.tlp, self.u = d(wl.tlp, torch.int32), d(wl.u, torch.float32)
        B = wl.B
        self.ids = torch.empty(B, dtype=torch.int32, device=dev)
        self.lp = torch.empty(B, dtype=torch.float32, device=dev)
        self.K = wl.K_max
        self.tids = torch.empty((B, max(self.K, 1)), dtype=torch.int32, device=dev)
        self.tlpo = torch.empty((B, max(self.K, 1)), dtype=torch.float32, device=dev)
        self.code = {"f32": 0, "bf16": 1, "f16": 2}[wl.dtype]
        from mlxforge_amd import _lib
        self.ws_bytes = _lib.workspace_size(B, wl.V, self.K, self.code)
        self.ws = torch.zeros(self.ws_bytes, dtype=torch.uint8, device=dev)
        self.stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        P = ctypes.c_void_p
        self.args_tail = [P(self.T.data_ptr()), P(self.k.data_ptr()), P(self.p.data_ptr()),
                          P(self.tlp.data_ptr()), P(self.u.data_ptr()), P(self.ids.data_ptr()),
                          P(self.lp.data_ptr()),
                          P(self.tids.data_ptr()) if self.K else None,
                          P(self.tlpo.data_ptr()) if self.K else None, self.K,
                          P(self.ws.data_ptr()), self.ws_bytes, self.stream]
        self.row_bytes = wl.V * wl.elem_size
        self.i = 0
        # refine stages from the host-side parameters (what a serving loop
        # knows about its rows); unhinted = the generic mlxf_sample path
        self.stages = _lib.refine_stages(B, wl.V, self.code, wl.T, wl.k, wl.p) if hinted else 3

    def _logits(self):
        p = self.buf[self.i % self.R].data_ptr()
        self.i += 1
        return ctypes.c_void_p(p)

    def run(self):
        err = ctypes.c_void_p()
        rc = self.lib.mlxf_sample_staged(self._logits(), self.code, self.wl.B, self.wl.V, self.wl.V,
                                         *self.args_tail[:-1], self.stages, self.args_tail[-1],
                                         ctypes.byref(err))
        if rc:
            from mlxforge_amd import _lib
            _lib.check(rc, err)


class MaskedStep(Step):
    """A grammar-constrained decode step (src/runtime/worker.cpp:142-179, 455-459):
    mlxf_apply_mask turns the bf16 rows and a bit mask (one bit per token, half
    of the tokens allowed, seeded) into fp32 rows, which mlxf_sample_staged then
    samples as fp32 logits."""

    def __init__(self, wl, torch, lib, frac=0.5):
        import numpy as np
        super().__init__(wl, torch, lib)
        dev = torch.device("cuda:0")
        rng = np.random.default_rng(0xB175)
        allowed = rng.random((wl.B, wl.V)) < frac
        nw = (wl.V + 31) // 32
        packed = np.zeros((wl.B, nw * 32), np.uint8)
        packed[:, :wl.V] = allowed
        words = np.packbits(packed.reshape(wl.B, nw, 4, 8)[:, :, :, ::-1], axis=-1).reshape(wl.B, nw, 4)
        bits = (words[:, :, 0].astype(np.uint32) | (words[:, :, 1].astype(np.uint32) << 8)
                | (words[:, :, 2].astype(np.uint32) << 16) | (words[:, :, 3].astype(np.uint32) << 24))
        self.bits = torch.from_numpy(bits.view(np.int32)).to(dev)
        self.nw = nw
        self.masked = torch.empty((wl.B, wl.V), dtype=torch.float32, device=dev)
        from mlxforge_amd import _lib
        self.ws_bytes_f32 = _lib.workspace_size(wl.B, wl.V, self.K, 0)
        self.ws32 = torch.zeros(self.ws_bytes_f32, dtype=torch.uint8, device=dev)
        self.stages32 = _lib.refine_stages(wl.B, wl.V, 0, wl.T, wl.k, wl.p)
        self.mask_only = False

    def run(self):
        err = ctypes.c_void_p()
        P = ctypes.c_void_p
        rc = self.lib.mlxf_apply_mask(self._logits(), self.code, self.wl.B, self.wl.V, self.wl.V,
                                      P(self.bits.data_ptr()), self.nw, P(self.masked.data_ptr()),
                                      self.wl.V, self.stream, ctypes.byref(err))
        if rc == 0 and not self.mask_only:
            tail = list(self.args_tail)
            tail[-3], tail[-2] = P(self.ws32.data_ptr()), self.ws_bytes_f32
            rc = self.lib.mlxf_sample_staged(P(self.masked.data_ptr()), 0, self.wl.B, self.wl.V, self.wl.V,
                                             *tail[:-1], self.stages32, tail[-1], ctypes.byref(err))
        if rc:
            from mlxforge_amd import _lib
            _lib.check(rc, err)


def time_first_pass(step, torch, warmup, steps):
    """Average duration of the step's dominant kernel (k_scan1, the one HBM read
    of the logits) alone, from hipEvents around K back-to-back launches on the
    stream the library launches on (torch's current stream).  (An event pair
    around each launch adds the events' own cost to every launch: 11.8 us
    against the 9.7 us kernel-trace median on C3.)"""
    def one():
        err = ctypes.c_void_p()
        rc = step.lib.mlxf_sampler_first_pass(step._logits(), step.code, step.wl.B, step.wl.V,
                                              step.wl.V, *step.args_tail, ctypes.byref(err))
        if rc:
            from mlxforge_amd import _lib
            _lib.check(rc, err)
    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        one()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_steps(step, torch, warmup, steps):
    for _ in range(warmup):
        step.run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step.run()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(wl, seconds):
    """The CPU restatement of the reference sampler (oracle/, reference-shaped:
    full-vocab sorts for top-p and top_logprobs) on the same decode step, built
    -O3 -march=native on this host, timed on the host threads this job may use
    (at most 16: the CPU share of one GPU on the box) and single-threaded."""
    import tempfile

    from oracle import oracle as orc
    code = {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}[wl.dtype]
    nproc = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = nproc
    threads = max(1, min(avail, 16))
    out_dir = tempfile.mkdtemp(prefix="mlxf_oracle_native_")
    L = orc.native_lib(out_dir)

    def timed(nthreads, budget):
        orc.sample(wl.logits[:1], T=wl.T[:1], k=wl.k[:1], p=wl.p[:1], tlp=wl.tlp[:1], u=wl.u[:1],
                   K_max=wl.K_max, dtype=code, nthreads=1, L=L)  # load + warm
        times = []
        t_end = time.perf_counter() + budget
        while True:
            t0 = time.perf_counter()
            orc.sample(wl.logits, T=wl.T, k=wl.k, p=wl.p, tlp=wl.tlp, u=wl.u, K_max=wl.K_max,
                       dtype=code, nthreads=nthreads, L=L)
            times.append(time.perf_counter() - t0)
            if time.perf_counter() >= t_end and len(times) >= 3:
                break
        times.sort()
        return times[len(times) // 2], len(times)

    med, reps = timed(threads, seconds * 0.6)
    med1, reps1 = timed(1, seconds * 0.4)
    return {"value": round(wl.B / med, 2), "unit": "rows/s", "cores": threads, "kind": "port",
            "sample": f"median of {reps} full decode steps of {wl.name} on {threads} threads "
                      f"(and of {reps1} single-threaded), oracle/sampler_oracle.c built "
                      f"-O3 -march=native on this host",
            "us_per_step": round(med * 1e6, 1), "us_per_step_1t": round(med1 * 1e6, 1),
            "rows_per_s_1t": round(wl.B / med1, 2), "threads": threads, "nproc": nproc,
            "affinity_cpus": avail, "cpu_model": _cpu_model(),
            "thread_cap": "16 = the host CPU share of one GPU on this box"}


def parity_report(step, torch):
    """One decode step of the timed configuration read back and checked against
    the oracle: every row must be the oracle's id or, for a row whose top-p
    cutoff, min_p threshold or draw boundary lies within 1e-6 (the exclusion
    rule), one of the ids that row admits when p, u and min_p move by 1e-6."""
    from oracle import oracle as orc
    wl = step.wl
    code = {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}[wl.dtype]
    step.i = 0
    step.run()
    torch.cuda.synchronize()
    ids = step.ids.cpu().numpy()
    o = orc.sample(wl.logits, T=wl.T, k=wl.k, p=wl.p, tlp=wl.tlp, u=wl.u, K_max=wl.K_max, dtype=code)
    rep = orc.check_rows(ids, o, wl.logits, code, T=wl.T, k=wl.k, p=wl.p, u=wl.u)
    rep["bad"] = len(rep["bad"])
    rep["exact"] = int((ids == o["ids"]).sum())
    return rep


def helpers_line(steps, warmup):
    """Microseconds per call of the calls around the decode step: the filter
    helpers (apply_top_k / apply_top_p / apply_min_p / filter_logits) and the
    sampling call with top_logprobs above the 64-entry lists, at B=64,
    V=151936 on N(0, 4^2) logits (fp32 and bf16), timed with events on
    torch's current stream."""
    import torch
    from mlxforge_amd import sampler
    B, V = 64, 151936
    g = torch.Generator(device="cuda").manual_seed(64)

    def t(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return round(e0.elapsed_time(e1) * 1000 / steps, 1)

    res = {}
    for name, dt in (("f32", torch.float32), ("bf16", torch.bfloat16)):
        x = (torch.randn(B, V, device="cuda", generator=g) * 4).to(dt)
        out = torch.empty_like(x)
        T = torch.full((B,), 0.8, device="cuda")
        k = torch.full((B,), 50, dtype=torch.int32, device="cuda")
        p = torch.full((B,), 0.9, device="cuda")
        mp = torch.full((B,), 0.05, device="cuda")
        u = torch.rand(B, device="cuda", generator=g)
        r = {"apply_top_k(50)": t(lambda: sampler.apply_top_k(x, 50, out=out)),
             "apply_top_p(0.9)": t(lambda: sampler.apply_top_p(x, 0.9, out=out)),
             "apply_min_p(0.05)": t(lambda: sampler.apply_min_p(x, 0.05, out=out)),
             "filter_logits(T=0.8,k=50,p=0.9,min_p=0.05)": t(lambda: sampler.filter_logits(
                 x, temperature=T, top_k=k, top_p=p, min_p=mp, out=out))}
        for K in (20, 65, 256, 4096):
            tl = torch.full((B,), K, dtype=torch.int32, device="cuda")
            r[f"sample_rows(T=0.8,p=0.9,top_logprobs={K})"] = t(lambda: sampler.sample_rows(
                x, temperature=T, top_p=p, top_logprobs=tl, uniforms=u, K_max=K, refine_stages=2))
        res[name] = r
    print(json.dumps({"helpers_us_per_call": res, "B": B, "V": V, "steps": steps, "warmup": warmup,
                      "data": "synthetic N(0, 4^2) logits"}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the other configs' lines")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run five plain 256 MiB device copies (counter scale factors)")
    ap.add_argument("--helpers", action="store_true",
                    help="only time the filter calls and wide top_logprobs (B=64, V=151936; one JSON line)")
    args = ap.parse_args()
    if args.helpers:
        helpers_line(args.steps, args.warmup)
        return
    if args.copy_calibration:
        import torch
        x = torch.ones(COPY_CALIBRATION_BYTES // 4, device="cuda")
        y = torch.empty_like(x)
        for _ in range(5):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": COPY_CALIBRATION_BYTES, "copies": 5}), flush=True)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); rows are independent, so N GPUs would each run this "
              f"same step on B/N rows with no communication.", file=sys.stderr)
        sys.exit(2)

    import torch

    from mlxforge_amd import _lib, workloads
    lib = _lib.load()
    assert torch.cuda.is_available(), "bench.py needs a GPU"

    parity = {}

    def measure(cfg, steps, warmup):
        wl = workloads.make(cfg)
        st = Step(wl, torch, lib)
        parity[f"C{cfg}"] = parity_report(st, torch)
        ms = time_steps(st, torch, warmup, steps)
        # the generic call (mlxf_sample: two refine stages, for a caller without
        # the parameters on the host) and all three stages
        st.stages, stages = 2, st.stages
        ms_gen = time_steps(st, torch, warmup, steps)
        st.stages = 3
        ms_all = time_steps(st, torch, warmup, steps)
        ms_k1 = time_first_pass(st, torch, warmup, steps)
        st_hot = Step(wl, torch, lib, rotate=False)
        ms_hot = time_steps(st_hot, torch, warmup, steps)
        del st, st_hot
        torch.cuda.empty_cache()
        return wl, ms, ms_hot, ms_all, stages, ms_k1, ms_gen

    log(f"[bench] config C{args.config}: warmup {args.warmup}, steps {args.steps}")
    wl, ms, ms_hot, ms_all, stages, ms_k1, ms_gen = measure(args.config, args.steps, args.warmup)
    alg = wl.algorithmic_bytes()
    # the dominant kernel, k_scan1, makes the step's one read of the logits; its
    # algorithmic bytes are the step's (logits read once, ids / logprobs / top-K
    # written, per-row parameters read) and its duration is timed alone
    achieved = alg / (ms_k1 * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(wl.B / (ms * 1e-3), 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"f32": "f32", "bf16": "bf16", "f16": "f16"}[wl.dtype],
        "data": "synthetic (seeded numpy PCG64 logits and uniforms, mlxforge_amd/workloads.py)",
        "config": {"workload": wl.name, "B": wl.B, "V": wl.V,
                   "logits_dtype": wl.dtype, "input_rotation": "cold (>512 MB of copies)"},
        "us_per_step": round(ms * 1e3, 2),
        "us_per_step_hot": round(ms_hot * 1e3, 2),
        "refine_stages": stages,
        "us_per_step_generic": round(ms_gen * 1e3, 2),
        "us_per_step_all_stages": round(ms_all * 1e3, 2),
        "achieved_GBps_step": round(alg / (ms * 1e-3) / 1e9, 1),
        "roofline": {"bound": "hbm", "kernel": "k_scan1", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": MEASURED_TRAFFIC_BYTES.get(args.config),
                     "algorithmic_bytes_per_launch": alg,
                     "kernel_us": round(ms_k1 * 1e3, 2)},
    }
    if not args.no_cpu:
        log("[bench] cpu baseline")
        out["cpu_baseline"] = cpu_baseline(wl, args.cpu_seconds)
    if not args.no_extra:
        extra = {}
        for cfg in (1, 2, 3, 4, 5):
            if cfg == args.config:
                continue
            log(f"[bench] extra config C{cfg}")
            w2, m2, mh2, ma2, st2, mk2, mg2 = measure(cfg, min(args.steps, 100), min(args.warmup, 10))
            extra[f"C{cfg}"] = {"workload": w2.name, "us_per_step": round(m2 * 1e3, 2),
                                "us_per_step_hot": round(mh2 * 1e3, 2),
                                "refine_stages": st2, "us_per_step_generic": round(mg2 * 1e3, 2),
                                "us_per_step_all_stages": round(ma2 * 1e3, 2),
                                "k_scan1_us": round(mk2 * 1e3, 2),
                                "rows_per_s": round(w2.B / (m2 * 1e-3), 1),
                                "achieved_GBps_step": round(w2.algorithmic_bytes() / (m2 * 1e-3) / 1e9, 1),
                                "hbm_frac": round(w2.algorithmic_bytes() / (m2 * 1e-3) / 1e9
                                                  / HBM_PEAK_GBPS, 4)}
        log("[bench] masked C2 step")
        ms_m = MaskedStep(workloads.make(2), torch, lib)
        m_step = time_steps(ms_m, torch, min(args.warmup, 10), min(args.steps, 100))
        ms_m.mask_only = True
        m_mask = time_steps(ms_m, torch, min(args.warmup, 10), min(args.steps, 100))
        w2 = ms_m.wl
        extra["C2_masked"] = {"workload": w2.name + " with a grammar bit mask (half the tokens allowed): "
                                          "mlxf_apply_mask to fp32 rows, then sampled as fp32",
                              "us_per_step": round(m_step * 1e3, 2), "us_mask_kernel": round(m_mask * 1e3, 2),
                              "refine_stages": ms_m.stages32,
                              "mask_GBps": round((w2.B * w2.V * (2 + 4) + w2.B * ms_m.nw * 4) / (m_mask * 1e-3) / 1e9, 1)}
        del ms_m
        torch.cuda.empty_cache()
        out["other_configs"] = extra
    out["parity_excluded"] = parity
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
