"""Seeded synthetic problems for the five BASELINE configurations (C1..C5).

Every problem is a single-level layer in this package's layout (groups of ``pool`` neurons,
slots = pool, no padding for the BASELINE pool sizes) with:
  * indices int32, K distinct per neuron, sorted ascending (sparse_pooling/layout.py:191-201);
  * weights fp32 N(0, 1/K), bias 0;
  * X and the upstream gradient dY N(0, 1) in the configuration's dtype.

C3 draws all indices of a pool from one contiguous 256-wide window at a random offset.
C5 draws 64 distinct candidates per neuron with envelope weights N(0, 1/16) and keeps the
top-16 |w| (stable descending order, ties to the lower candidate position), then stores the kept
(index, weight) pairs sorted by index: the per-neuron form of the Cover-TopK/16 support
selection (sparse_pooling/experimental/local_supports.py:209-222, 279-282).

``groups`` < the configuration's G gives a bounded sample of the same workload (same B, D,
pool size and fan-in, fewer pools), used for parity tests and the CPU baseline.
Generation is chunked and runs on ``device`` with a seeded torch.Generator; the same seed on the
same device type gives the same bits.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .layout import SparseLayout, sample_distinct

CONFIGS = {
    "C1": dict(B=64, D=1024, N=1_048_576, K=8, pool=256, x_dtype=torch.float32, indices="uniform",
               work="fwd+bwd+adam", note="CPU reference path shape"),
    "C2": dict(B=256, D=4096, N=100_663_296, K=8, pool=1024, x_dtype=torch.float32, indices="uniform",
               work="fwd", note="headline forward"),
    "C3": dict(B=256, D=4096, N=100_663_296, K=8, pool=1024, x_dtype=torch.bfloat16, indices="window256",
               work="fwd+bwd", note="locality windows of 256"),
    "C4": dict(B=1024, D=8192, N=100_663_296, K=8, pool=1024, x_dtype=torch.bfloat16, indices="uniform",
               work="fwd+bwd+adam", note="full training step"),
    "C5": dict(B=512, D=4096, N=50_331_648, K=16, pool=512, x_dtype=torch.float32, indices="top16of64",
               work="fwd+bwd_dx", note="per-neuron top-16 of a 64-candidate envelope"),
}
WINDOW = 256
CANDIDATES = 64


@dataclass
class Problem:
    name: str
    layout: SparseLayout
    idx: torch.Tensor      # [G, NB, 8, K] int32
    w: torch.Tensor        # [G, NB, 8, K] fp32
    b: torch.Tensor        # [G, NB, 8] fp32
    x: torch.Tensor        # [B, D]
    dy: torch.Tensor       # [B, G] fp32 values (bf16-exact for bf16 configs)
    pool: str = "sum"

    @property
    def B(self):
        return self.x.shape[0]

    @property
    def edges(self):
        return self.layout.hidden_dim * self.layout.fan_in


def _top_k_of_candidates(cand: torch.Tensor, wenv: torch.Tensor, k: int):
    """Keep the k largest |w| per row (stable: ties keep the lower candidate position), then
    order the kept pairs by index."""
    order = torch.sort(wenv.abs(), dim=1, descending=True, stable=True).indices[:, :k]
    ki = torch.gather(cand, 1, order)
    kw = torch.gather(wenv, 1, order)
    o2 = torch.sort(ki, dim=1).indices
    return torch.gather(ki, 1, o2), torch.gather(kw, 1, o2)


@torch.no_grad()
def make_problem(name: str, device="cpu", seed: int = 0, groups: int | None = None, batch: int | None = None,
                 chunk: int = 1 << 22) -> Problem:
    c = CONFIGS[name]
    B = batch if batch is not None else c["B"]
    D, K, pool = c["D"], c["K"], c["pool"]
    G = groups if groups is not None else c["N"] // pool
    N = G * pool
    L = SparseLayout(D, N, G, K, 8, False)
    assert L.slots_per_group == pool, "BASELINE pool sizes are multiples of 32"
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    idx = torch.empty((N, K), dtype=torch.int32, device=device)
    w = torch.empty((N, K), dtype=torch.float32, device=device)
    if c["indices"] == "uniform":
        for s in range(0, N, chunk):
            e = min(s + chunk, N)
            idx[s:e] = sample_distinct(e - s, D, K, gen, device).to(torch.int32)
        for s in range(0, N, chunk):
            e = min(s + chunk, N)
            w[s:e] = torch.randn((e - s, K), generator=gen, device=device) / math.sqrt(K)
    elif c["indices"] == "window256":
        off = torch.randint(0, D - WINDOW + 1, (G,), generator=gen, device=device, dtype=torch.int64)
        for s in range(0, N, chunk):
            e = min(s + chunk, N)
            rec = sample_distinct(e - s, WINDOW, K, gen, device)
            g = torch.arange(s, e, device=device) // pool
            idx[s:e] = (rec + off[g][:, None]).to(torch.int32)
        for s in range(0, N, chunk):
            e = min(s + chunk, N)
            w[s:e] = torch.randn((e - s, K), generator=gen, device=device) / math.sqrt(K)
    elif c["indices"] == "top16of64":
        for s in range(0, N, chunk // 4):
            e = min(s + chunk // 4, N)
            cand = sample_distinct(e - s, D, CANDIDATES, gen, device)
            wenv = torch.randn((e - s, CANDIDATES), generator=gen, device=device) / 4.0
            ki, kw = _top_k_of_candidates(cand, wenv, K)
            idx[s:e] = ki.to(torch.int32)
            w[s:e] = kw
    else:
        raise ValueError(c["indices"])
    b = torch.zeros((N,), dtype=torch.float32, device=device)
    xdt = c["x_dtype"]
    x = torch.randn((B, D), generator=gen, device=device).to(xdt)
    dy = torch.randn((B, G), generator=gen, device=device).to(xdt).to(torch.float32)
    return Problem(name, L, idx.view(L.index_shape), w.view(L.weight_shape), b.view(L.bias_shape), x, dy)
