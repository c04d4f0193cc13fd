"""Fused AdamW for the layer parameters, mirroring sparse_pooling/optim.py (FusedAdamW).

Reads the fp32 ``main_grad`` buffers written by the fused backward (or ``.grad``), updates the
parameters and zeroes the gradient in the same streaming pass (the HIP kernel gl_adam).
Semantics are dense AdamW for every element (optim.py:1-15): m = b1 m + (1-b1) g,
v = b2 v + (1-b2) g^2, p = p (1 - lr wd) - lr (m / bc1) / (sqrt(v / bc2) + eps), bc_i = 1 - b_i^t.

Moments are fp32 (``moments="fp32"``) or bf16 (``"bf16"``, the reference default).  Parameters
are fp32, or bf16 with the reference's three variants (optim.py:5-9, 52-62): an fp32 master copy
in the optimizer state (``master_weights=True``; the update runs on it and the parameter gets its
nearest-even rounding), stochastic rounding (the default without masters: noise from Triton's
``tl.randint(seed, element)`` below the bf16 cut, the seed counting launches as the reference's
``_seed`` does), or nearest-even rounding (``stochastic_rounding=False``).
"""
from __future__ import annotations

from typing import Iterable

import torch

from .backend import backend_for


class FusedAdamW(torch.optim.Optimizer):
    def __init__(self, params: Iterable[torch.nn.Parameter], lr=1e-3, betas=(0.9, 0.999), eps=1e-8,
                 weight_decay=0.0, moments: str = "bf16", master_weights: bool = False,
                 stochastic_rounding: bool = True):
        if moments not in ("bf16", "fp32"):
            raise ValueError("moments must be 'bf16' or 'fp32'")
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay)
        super().__init__(params, defaults)
        self.moments = moments
        self.master_weights = master_weights
        self.stochastic_rounding = stochastic_rounding
        self._seed = 0

    def state_bytes(self) -> int:
        n = 0
        for st in self.state.values():
            for t in st.values():
                if torch.is_tensor(t):
                    n += t.numel() * t.element_size()
        return n

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        mdt = torch.bfloat16 if self.moments == "bf16" else torch.float32
        for group in self.param_groups:
            b1, b2 = group["betas"]
            for p in group["params"]:
                g = getattr(p, "main_grad", None)
                if g is None:
                    if p.grad is None:
                        continue
                    g = p.grad.float().contiguous()
                if p.dtype not in (torch.float32, torch.bfloat16):
                    raise NotImplementedError(f"FusedAdamW updates fp32 or bf16 parameters (got {p.dtype})")
                if not p.is_contiguous() or not g.is_contiguous():
                    raise ValueError("FusedAdamW needs contiguous parameters and gradients")
                st = self.state[p]
                if not st:
                    st["step"] = 0
                    st["m"] = torch.zeros(p.shape, device=p.device, dtype=mdt)
                    st["v"] = torch.zeros(p.shape, device=p.device, dtype=mdt)
                    if self.master_weights and p.dtype != torch.float32:
                        st["master"] = p.detach().float().clone()
                st["step"] += 1
                t = st["step"]
                self._seed += 1
                backend_for(p.device).adam(p, g, st["m"], st["v"], group["lr"], b1, b2, group["eps"],
                                           group["weight_decay"], 1 - b1 ** t, 1 - b2 ** t, master=st.get("master"),
                                           stochastic=self.stochastic_rounding, seed=self._seed)
                if getattr(p, "main_grad", None) is None:
                    p.grad = None
        return loss
