"""Semantic two-level pooling: y = level2(transform(level1(x))).

Level 1 pools each group's shards of ``neurons_per_shard`` slots on the HIP kernels (the shards are
the kernels' pooling units, ``Level1Runtime(..., nps)``), giving features F [B, G, S] with
S = ceil(max_group / neurons_per_shard).  Level 2 only ever touches F, so it runs as ordinary
PyTorch ops on the GPU, as in the reference (sparse_pooling/reference/pytorch_reference.py:107-125:
"shared by the reference and the production layer").

* ``apply_transform``  - pytorch_reference.py:110-122 (none | activation | affine | gate);
* ``pool_features``    - level-2 pooling of F's last dimension, every shard valid
                         (pytorch_reference.py:50-100 with an all-true mask);
* ``level2_forward``   - pytorch_reference.py:125-133 (weighted_sum with learned v, or a pool);
* ``SemanticPoolFunction`` - sparse_pooling/autograd.py:417-476: level-1 statistics kept from the
  forward (level1_checkpoint="save") or rebuilt by recomputation ("recompute"); backward takes
  dF by autograd through level 2 and hands g_pre = dF * out_act'(pre) to the level-1 backward.
"""
from __future__ import annotations

import math
from typing import Dict, List

import torch

from .autograd import (CHECKPOINT_BUDGET, Level1Runtime, _compute_operands, _grad_buffers, _ids_per_token,
                       _level1_backward, _saved_stats, act_torch, fit_policy)
from .config import LevelSpec, PoolingConfig


def apply_transform(f: torch.Tensor, level1: LevelSpec, tparams: Dict[str, torch.Tensor]) -> torch.Tensor:
    """The learned map between the levels, per (group, shard) (pytorch_reference.py:110-122)."""
    tr = level1.transform
    if tr == "none":
        return f
    if tr == "activation":
        return act_torch(f, level1.transform_activation)
    if tr == "affine":
        return act_torch(tparams["alpha"] * f + tparams["beta"], level1.transform_activation)
    if tr == "gate":
        return f * torch.sigmoid(tparams["alpha"] * f + tparams["beta"])
    raise ValueError(f"unknown transform {tr!r}")


def _first_max(a: torch.Tensor) -> torch.Tensor:
    # the first maximum (smallest shard) takes the whole gradient, as argmax + gather does
    return a.gather(-1, torch.argmax(a, dim=-1, keepdim=True)).squeeze(-1)


def _topk_mean(h: torch.Tensor, a: torch.Tensor, k: int) -> torch.Tensor:
    # the k largest raw features (stable: ties to the smaller shard), mean of their activations
    kk = min(k, h.shape[-1])
    order = torch.sort(h.detach(), dim=-1, descending=True, stable=True).indices[..., :kk]
    return a.gather(-1, order).sum(-1) / kk


def _power_mean(a: torch.Tensor, p: float) -> torch.Tensor:
    # (mean a^p)^(1/p) of non-negative a, scaled by the largest value so a^p cannot overflow
    m = a.amax(-1, keepdim=True)
    safe = torch.where(m > 0, m, torch.ones_like(m))
    s = ((a / safe) ** p).mean(-1)
    return torch.where(m.squeeze(-1) > 0, safe.squeeze(-1) * s ** (1.0 / p), torch.zeros_like(s))


def pool_features(h: torch.Tensor, level: LevelSpec) -> torch.Tensor:
    """Pool the last dimension of h [B, G, S] (every entry valid) with a level's operator, then
    its out-activation (pytorch_reference.py:50-100)."""
    a = act_torch(h, level.activation)
    S = h.shape[-1]
    t = level.type
    if t == "max":
        pooled = _first_max(a)
    elif t == "topk_mean":
        pooled = _topk_mean(h, a, level.k)
    elif t == "mean":
        pooled = a.mean(-1)
    elif t == "sum":
        pooled = a.sum(-1)
    elif t == "logmeanexp":
        tau = level.temperature
        pooled = tau * (torch.logsumexp(a / tau, dim=-1) - math.log(S))
    elif t == "power_mean":
        pooled = _power_mean(a, level.p)
    elif t == "softmax_weighted":
        pooled = (torch.softmax(level.beta * a, dim=-1) * a).sum(-1)
    else:
        raise ValueError(f"{t!r} is not a level-2 pool")
    return act_torch(pooled, level.out_activation)


def level2_forward(f: torch.Tensor, cfg: PoolingConfig, tparams: Dict[str, torch.Tensor]) -> torch.Tensor:
    """F [B, G, S] level-1 features -> y [B, G] (pytorch_reference.py:125-133)."""
    l1, l2 = cfg.levels
    h = apply_transform(f, l1, tparams)
    if l2.type == "weighted_sum":
        return act_torch((h * tparams["v"]).sum(-1), l2.out_activation)
    return pool_features(h, l2)


class SemanticPoolFunction(torch.autograd.Function):
    """Two-level: F = out_act(level1(x)) [B, G, S]; y = level2(transform(F)) (autograd.py:417-476).

    level1_checkpoint "save": pre (and the level-1 statistics the policy keeps) saved by the
    forward; "recompute": only x / W / b, the backward reruns the level-1 forward."""

    @staticmethod
    def forward(ctx, x, w, b, rt: Level1Runtime, cfg: PoolingConfig, policy: str, compute_dtype,
                tnames: List[str], *tparams):
        policy = fit_policy(rt, policy, x.shape[0])
        xc, wc, bc = _compute_operands(x, w, b, compute_dtype)
        l1 = rt.level
        out = rt.forward(xc, wc, bc, track_ids=(policy == "save_winners"))
        B = x.shape[0]
        G, S = rt.layout.groups, rt.units.S
        F = act_torch(out["pre"], l1.out_activation).reshape(B, G, S)
        tp = dict(zip(tnames, tparams))
        with torch.no_grad():
            y = level2_forward(F, cfg, tp)
        if cfg.level1_checkpoint == "save":
            saved = _saved_stats(l1, out, policy if policy != "recompute_stats" else "minimal_stats")
        else:
            saved = {}
        ctx.rt, ctx.cfg, ctx.policy, ctx.compute_dtype, ctx.tnames = rt, cfg, policy, compute_dtype, tnames
        ctx.saved_keys = list(saved.keys())
        ctx.n_t = len(tparams)
        ctx.save_for_backward(x, w, b, *tparams, *saved.values())
        rt.last_info["checkpoint_bytes"] = sum(t.numel() * t.element_size() for t in saved.values())
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, b, *rest = ctx.saved_tensors
        tparams = rest[: ctx.n_t]
        saved = dict(zip(ctx.saved_keys, rest[ctx.n_t:]))
        rt: Level1Runtime = ctx.rt
        l1 = rt.level
        xc, wc, bc = _compute_operands(x, w, b, ctx.compute_dtype)
        rebuilt = "pre" not in saved
        B = x.shape[0]
        if rebuilt:
            # level1_checkpoint="recompute": rebuild the level-1 features, with the selected slots a
            # max / top-k level 1 needs when they fit the checkpoint budget (otherwise the level-1
            # backward recomputes them one token chunk at a time)
            track = l1.type in ("max", "topk_mean") and B * _ids_per_token(rt) * 4 <= CHECKPOINT_BUDGET
            saved.update(rt.forward(xc, wc, bc, track_ids=track))
        G, S = rt.layout.groups, rt.units.S
        pre = saved["pre"]
        with torch.enable_grad():
            Fv = act_torch(pre, l1.out_activation).reshape(B, G, S).detach().requires_grad_(True)
            tp = [p.detach().requires_grad_(True) for p in tparams]
            y = level2_forward(Fv, ctx.cfg, dict(zip(ctx.tnames, tp)))
            grads = torch.autograd.grad(y, [Fv] + tp, dy, allow_unused=True)
        dF = grads[0].reshape(B, G * S)
        policy = ctx.policy if ctx.policy != "recompute_stats" else "minimal_stats"
        dw_buf, db_buf, use_main = _grad_buffers(w, b)
        dx = _level1_backward(rt, xc, wc, bc, dF, saved, policy, dw_buf, db_buf, rebuilt)
        gw = None if use_main else dw_buf.to(w.dtype)
        gb = None if use_main else db_buf.to(b.dtype)
        return (dx.to(x.dtype, memory_format=torch.contiguous_format), gw, gb, None, None, None, None, None,
                *grads[1:])
