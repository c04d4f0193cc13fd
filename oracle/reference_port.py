"""TEST INFRASTRUCTURE ONLY: the reference's materialising CPU path, restated in PyTorch, used as
bench.py's ``cpu_baseline`` (kind "port").  Never imported by the product package.

One training step of a single-level Mode-A layer, the way sparse_pooling/reference computes it:
  xg = x[:, idx]  [B, N, K] gather          pytorch_reference.py:43-44
  z  = (xg * w).sum(-1) + b                 pytorch_reference.py:45-46
  a  = relu(z); pooled = masked sum (/ n_g for mean) over each group   pytorch_reference.py:50-79
  autograd for dX, dW, db; torch.optim.Adam(lr, betas, eps) fp32      (SURVEY 8(d) CPU baseline)
"""
from __future__ import annotations

import time

import torch


class PortStep:
    def __init__(self, idx, w, b, counts, S, pool="sum", lr=1e-3, betas=(0.9, 0.999), eps=1e-8):
        self.idx = idx.reshape(-1, idx.shape[-1]).long()
        self.w = torch.nn.Parameter(w.reshape(self.idx.shape).float().clone())
        self.b = torch.nn.Parameter(b.reshape(-1).float().clone())
        self.counts = counts.long()
        self.S = S
        self.G = len(counts)
        self.pool = pool
        self.valid = (torch.arange(S)[None, :] < self.counts[:, None]).reshape(-1)
        self.opt = torch.optim.Adam([self.w, self.b], lr=lr, betas=betas, eps=eps)

    def forward(self, x):
        xg = x[:, self.idx]
        z = (xg * self.w[None]).sum(-1) + self.b[None]
        a = torch.relu(z) * self.valid
        s = a.reshape(x.shape[0], self.G, self.S).sum(-1)
        return s / self.counts if self.pool == "mean" else s

    def step(self, x, dy):
        x = x.detach().requires_grad_(True)
        t0 = time.perf_counter()
        y = self.forward(x)
        t1 = time.perf_counter()
        (y * dy).sum().backward()
        t2 = time.perf_counter()
        self.opt.step()
        self.opt.zero_grad(set_to_none=True)
        t3 = time.perf_counter()
        return {"fwd": t1 - t0, "bwd": t2 - t1, "adam": t3 - t2, "step": t3 - t0}
