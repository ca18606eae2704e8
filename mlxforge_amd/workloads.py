"""Seeded synthetic decode-step inputs for the five benchmark configurations.

Each config is one decode step of the sampler: a [B, V] logits matrix plus the
per-row parameters and uniforms.  Inputs are generated on the host with numpy's
PCG64 (seed 0x5EED0000 + config number), so the GPU path and the CPU baseline
see bit-identical data.  bf16 logits are produced by round-to-nearest-even and
returned as uint16 bit patterns.

  C1 greedy + chosen logprob, B=1,   V=128256, fp32 N(0, 2^2), 5 indices +10
  C2 T=0.7, top-p 0.9,        B=8,   V=151936, bf16 3*N(0,1), 20 indices + U(4,9)
  C3 T=1, top-k 50, p=0.95,   B=32,  V=151936, fp32 2.5*Gumbel - 1.1*ln(i+1);
                                     rows r%4==0 repeat their max at a second index
  C4 top_logprobs=20,         B=64,  V=151936, fp32 N(0, 4^2), T~U(.3,1.5), p~U(.5,1)
  C5 mixed batch,             B=256, V=262144, bf16: 51 greedy, 103 top-k
                                     (k cycles 1,20,100,1000), 102 top-p (p cycles
                                     .8,.95,1); T~U(.5,1.2); half peaked rows
                                     (N(0,3^2), one index = 15), half flat N(0,.1^2)
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

SEED_BASE = 0x5EED0000


@dataclass
class Workload:
    name: str
    B: int
    V: int
    dtype: str            # "f32" | "bf16"
    logits: np.ndarray    # float32 [B, V] or uint16 bf16 bits [B, V]
    T: np.ndarray         # float32 [B]
    k: np.ndarray         # int32 [B]
    p: np.ndarray         # float32 [B]
    tlp: np.ndarray       # int32 [B]
    u: np.ndarray         # float32 [B]
    K_max: int

    @property
    def elem_size(self) -> int:
        return 4 if self.dtype == "f32" else 2

    def algorithmic_bytes(self) -> int:
        """One compulsory read of the logits + ids and chosen logprobs + top-K
        pairs + per-row parameters and uniform."""
        return (self.B * self.V * self.elem_size + self.B * 8 + self.B * self.K_max * 8
                + self.B * 16)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    u = u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))
    return (u >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def _c1(rng):
    B, V = 1, 128256
    z = rng.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)
    idx = rng.choice(V, 5, replace=False)
    z[0, idx] += np.float32(10.0)
    return Workload("C1 greedy+logprob B=1 V=128256 f32", B, V, "f32", z,
                    np.zeros(B, np.float32), np.zeros(B, np.int32), np.ones(B, np.float32),
                    np.zeros(B, np.int32), np.zeros(B, np.float32), 0)


def _c2(rng):
    B, V = 8, 151936
    z = rng.standard_normal((B, V), dtype=np.float32) * np.float32(3.0)
    for r in range(B):
        idx = rng.choice(V, 20, replace=False)
        z[r, idx] += rng.uniform(4.0, 9.0, 20).astype(np.float32)
    return Workload("C2 T=0.7 top-p=0.9 B=8 V=151936 bf16", B, V, "bf16", to_bf16_bits(z),
                    np.full(B, 0.7, np.float32), np.zeros(B, np.int32),
                    np.full(B, 0.9, np.float32), np.full(B, -1, np.int32),
                    rng.random(B, dtype=np.float32), 0)


def _c3(rng):
    B, V = 32, 151936
    uni = rng.random((B, V), dtype=np.float32)
    uni = np.clip(uni, np.float32(1e-30), np.float32(1.0 - 2.0 ** -24))
    gumbel = -np.log(-np.log(uni))
    prior = np.float32(1.1) * np.log(np.arange(1, V + 1, dtype=np.float32))
    z = (np.float32(2.5) * gumbel - prior[None, :]).astype(np.float32)
    for r in range(0, B, 4):
        am = int(np.argmax(z[r]))
        j = int(rng.integers(V))
        while j == am:
            j = int(rng.integers(V))
        z[r, j] = z[r, am]
    return Workload("C3 T=1 top-k=50 top-p=0.95 B=32 V=151936 f32", B, V, "f32", z,
                    np.ones(B, np.float32), np.full(B, 50, np.int32),
                    np.full(B, 0.95, np.float32), np.full(B, -1, np.int32),
                    rng.random(B, dtype=np.float32), 0)


def _c4(rng):
    B, V = 64, 151936
    z = rng.standard_normal((B, V), dtype=np.float32) * np.float32(4.0)
    T = rng.uniform(0.3, 1.5, B).astype(np.float32)
    p = rng.uniform(0.5, 1.0, B).astype(np.float32)
    return Workload("C4 top_logprobs=20 B=64 V=151936 f32", B, V, "f32", z, T,
                    np.zeros(B, np.int32), p, np.full(B, 20, np.int32),
                    rng.random(B, dtype=np.float32), 20)


def _c5(rng):
    B, V = 256, 262144
    roles = np.array([0] * 51 + [1] * 103 + [2] * 102)
    rng.shuffle(roles)
    T = np.zeros(B, np.float32)
    k = np.zeros(B, np.int32)
    p = np.ones(B, np.float32)
    ks, ps = [1, 20, 100, 1000], [0.8, 0.95, 1.0]
    nk = npp = 0
    for r in range(B):
        if roles[r] == 0:
            continue
        T[r] = np.float32(rng.uniform(0.5, 1.2))
        if roles[r] == 1:
            k[r] = ks[nk % 4]
            nk += 1
        else:
            p[r] = ps[npp % 3]
            npp += 1
    peaked = rng.random(B) < 0.5
    z = rng.standard_normal((B, V), dtype=np.float32)
    z[peaked] *= np.float32(3.0)
    z[~peaked] *= np.float32(0.1)
    for r in np.nonzero(peaked)[0]:
        z[r, int(rng.integers(V))] = np.float32(15.0)
    return Workload("C5 mixed B=256 V=262144 bf16", B, V, "bf16", to_bf16_bits(z), T, k, p,
                    np.full(B, -1, np.int32), rng.random(B, dtype=np.float32), 0)


_MAKERS = {1: _c1, 2: _c2, 3: _c3, 4: _c4, 5: _c5}


def make(config: int) -> Workload:
    """Config 1..5, deterministic."""
    return _MAKERS[config](np.random.default_rng(SEED_BASE + config))
