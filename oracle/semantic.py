"""TEST INFRASTRUCTURE ONLY: CPU oracle of semantic two-level pooling, float64.

Only ``tests/`` may import this module, and only as the checker.

* Level 1 (``level1_forward`` / ``level1_backward``): every group's shards of ``nps`` slots are the
  pooling units (sparse_pooling/kernels/ops.py:45-56, pytorch_reference.py:136-148 shard_view):
  unit u = g * S + s pools slots [s * nps, s * nps + counts[u]) of group g.  The shards are copied
  into a layout of their own (one pool of nps slots per shard, padding zeroed) and the level-1 C
  oracle (oracle.py, gl_oracle.c) runs on it; gradients are scattered back to the group layout.
* Level 2 (``level2_forward`` / ``level2_backward``): numpy restatement of
  pytorch_reference.py:110-133 (transforms none | activation | affine | gate; weighted_sum or a
  pool of the S shard features, every shard valid, pytorch_reference.py:50-100), with the
  gradients derived by hand (no autograd).

Parity status (tests/test_semantic.py):
  level1_*   pinned: Sum -> Sum with identity activations equals the flat sum over the group
             (forward and gradients, any shard sizes); Mean -> Mean equals the flat mean when every
             shard is full and differs with a partial last shard (test_hierarchical_pooling.py:104-115);
             Max -> Max equals the flat maximum (test_hierarchical_pooling.py:97-101).
  level2_*   pinned: float64 central differences of level2_forward for every transform and level-2
             operator; weighted_sum with v = 1/S equals mean; one shard reduces to the level-2
             activations of that feature.
"""
from __future__ import annotations

import math

import numpy as np

from . import oracle as O

# ----------------------------------------------------------------------------- level 1


def shard_units(counts, nps: int):
    """(S, counts_u [G * S]) of groups with counts [G] cut into shards of nps slots."""
    counts = np.asarray(counts, np.int64)
    S = int(math.ceil(counts.max() / nps))
    s = np.arange(S)
    cnt = np.clip(counts[:, None] - s[None, :] * nps, 0, nps)
    if (cnt == 0).any():
        raise ValueError("a semantic shard would be empty")
    return S, cnt.reshape(-1).astype(np.int32)


def _shard_rows(counts, gs: int, nps: int):
    """rows [G * S * nps] of the group layout behind each shard slot (-1: padding), counts_u."""
    S, cu = shard_units(counts, nps)
    G = len(counts)
    u = np.arange(G * S)
    g, sh = u // S, u % S
    sl = np.arange(nps)
    rows = g[:, None] * gs + sh[:, None] * nps + sl[None, :]
    rows = np.where(sl[None, :] < cu[:, None], rows, -1)
    return S, cu, rows.reshape(-1)


def _virtual(idx, w, bias, counts, gs: int, nps: int):
    S, cu, rows = _shard_rows(counts, gs, nps)
    K = idx.shape[1]
    ok = rows >= 0
    r = np.where(ok, rows, 0)
    vi = np.where(ok[:, None], np.asarray(idx).reshape(-1, K)[r], 0).astype(np.int32)
    vw = np.where(ok[:, None], np.asarray(w, np.float32).reshape(-1, K)[r], 0).astype(np.float32)
    vb = np.where(ok, np.asarray(bias, np.float32).reshape(-1)[r], 0).astype(np.float32)
    return S, cu, rows, vi, vw, vb


def level1_forward(x, idx, w, bias, counts, gs: int, nps: int, level):
    """Level-1 pooled values of every shard: (pre [B, G * S] float64, mag [B, G * S] error scale,
    sel: the selected shard slots for max / top-k mean, else None)."""
    S, cu, rows, vi, vw, vb = _virtual(idx, w, bias, counts, gs, nps)
    t, act = level.type, level.activation
    if t in ("mean", "sum"):
        pre, mag = O.forward(x, vi, vw, vb, cu, nps, act=act, pool=t, with_mag=True)
        return pre, mag, None
    if t == "max":
        pre, win, _ = O.forward_max(x, vi, vw, vb, cu, nps, act=act)
        return pre, np.abs(pre), win
    if t == "topk_mean":
        pre, slots, _ = O.forward_topk(x, vi, vw, vb, cu, nps, level.k, act=act)
        return pre, np.abs(pre), slots
    param = {"logmeanexp": level.temperature, "power_mean": level.p, "softmax_weighted": level.beta}[t]
    pre, _, mag = O.forward_smooth(x, vi, vw, vb, cu, nps, t, param, act=act)
    return pre, mag, None


def level1_backward(x, idx, w, bias, counts, gs: int, nps: int, level, g_pre):
    """(dW, db, dX) float64 in the group layout for g_pre [B, G * S], the gradient of every shard's
    pooled value."""
    S, cu, rows, vi, vw, vb = _virtual(idx, w, bias, counts, gs, nps)
    t, act = level.type, level.activation
    if t in ("mean", "sum"):
        vW, vB, dX = O.backward(x, vi, vw, vb, cu, nps, g_pre, act=act, pool=t)
    elif t == "max":
        _, win, _ = O.forward_max(x, vi, vw, vb, cu, nps, act=act)
        vW, vB, dX, _ = O.backward_events(x, vi, vw, vb, cu, nps, g_pre, win, act=act)
    elif t == "topk_mean":
        vW, vB, dX = O.backward_topk(x, vi, vw, vb, cu, nps, g_pre, level.k, act=act)
    else:
        param = {"logmeanexp": level.temperature, "power_mean": level.p, "softmax_weighted": level.beta}[t]
        vW, vB, dX, _ = O.backward_smooth(x, vi, vw, vb, cu, nps, g_pre, t, param, act=act)
    K = np.asarray(idx).shape[-1]
    n = np.asarray(bias).size
    dW = np.zeros((n, K), np.float64)
    db = np.zeros(n, np.float64)
    ok = rows >= 0
    dW[rows[ok]] = vW[ok]
    db[rows[ok]] = vB[ok]
    return dW, db, dX


# ----------------------------------------------------------------------------- level 2

_SQRT1_2 = 1.0 / math.sqrt(2.0)


def _erf(x):
    return np.vectorize(math.erf, otypes=[np.float64])(x)


def act(x, name):
    if name == "identity":
        return x
    if name == "relu":
        return np.maximum(x, 0.0)
    if name == "gelu":
        return 0.5 * x * (1.0 + _erf(x * _SQRT1_2))
    raise ValueError(name)


def dact(x, name):
    if name == "identity":
        return np.ones_like(x)
    if name == "relu":
        return (x > 0).astype(np.float64)
    if name == "gelu":
        return 0.5 * (1.0 + _erf(x * _SQRT1_2)) + x * np.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)
    raise ValueError(name)


def _sigmoid(u):
    return 1.0 / (1.0 + np.exp(-u))


def _transform(f, l1, tp):
    """h and the pieces its gradient needs."""
    tr = l1.transform
    if tr == "none":
        return f, None
    if tr == "activation":
        return act(f, l1.transform_activation), None
    u = tp["alpha"] * f + tp["beta"]
    if tr == "affine":
        return act(u, l1.transform_activation), u
    if tr == "gate":
        return f * _sigmoid(u), u
    raise ValueError(tr)


def _pool(h, l2):
    """(pooled before out-activation, dpooled/dh) of the last axis of h [B, G, S]."""
    a = act(h, l2.activation)
    da = dact(h, l2.activation)
    S = h.shape[-1]
    t = l2.type
    grad = np.zeros_like(h)
    if t == "max":
        j = np.argmax(a, axis=-1)  # first maximum
        pooled = np.take_along_axis(a, j[..., None], -1)[..., 0]
        np.put_along_axis(grad, j[..., None], 1.0, -1)
    elif t == "topk_mean":
        kk = min(l2.k, S)
        order = np.argsort(-h, axis=-1, kind="stable")[..., :kk]  # largest raw h, ties to the smaller shard
        pooled = np.take_along_axis(a, order, -1).sum(-1) / kk
        np.put_along_axis(grad, order, 1.0 / kk, -1)
    elif t == "mean":
        pooled = a.mean(-1)
        grad[:] = 1.0 / S
    elif t == "sum":
        pooled = a.sum(-1)
        grad[:] = 1.0
    elif t == "logmeanexp":
        tau = l2.temperature
        m = (a / tau).max(-1, keepdims=True)
        e = np.exp(a / tau - m)
        pooled = tau * (m[..., 0] + np.log(e.sum(-1)) - math.log(S))
        grad = e / e.sum(-1, keepdims=True)
    elif t == "power_mean":
        p = l2.p
        m = a.max(-1, keepdims=True)
        safe = np.where(m > 0, m, 1.0)
        r = a / safe
        s = (r ** p).mean(-1, keepdims=True)
        pooled = np.where(m[..., 0] > 0, safe[..., 0] * s[..., 0] ** (1.0 / p), 0.0)
        # d/da_i (mean a^p)^(1/p) = (mean r^p)^(1/p - 1) r_i^(p - 1) / S, scale-free in r = a / m
        grad = np.where(m > 0, s ** (1.0 / p - 1.0) * r ** (p - 1.0) / S, 0.0)
    elif t == "softmax_weighted":
        beta = l2.beta
        u = beta * a
        e = np.exp(u - u.max(-1, keepdims=True))
        pw = e / e.sum(-1, keepdims=True)
        pooled = (pw * a).sum(-1)
        grad = pw * (1.0 + beta * (a - pooled[..., None]))
    else:
        raise ValueError(t)
    return pooled, grad * da


def level2_forward(F, l1, l2, tparams):
    """y [B, G] float64 from level-1 features F [B, G, S] (pytorch_reference.py:125-133)."""
    F = np.asarray(F, np.float64)
    tp = {k: np.asarray(v, np.float64) for k, v in (tparams or {}).items()}
    h, _ = _transform(F, l1, tp)
    if l2.type == "weighted_sum":
        return act((h * tp["v"]).sum(-1), l2.out_activation)
    pooled, _ = _pool(h, l2)
    return act(pooled, l2.out_activation)


def level2_backward(F, l1, l2, tparams, dy):
    """(dF [B, G, S], {name: gradient [G, S]}) for upstream dy [B, G]."""
    F = np.asarray(F, np.float64)
    dy = np.asarray(dy, np.float64)
    tp = {k: np.asarray(v, np.float64) for k, v in (tparams or {}).items()}
    h, u = _transform(F, l1, tp)
    dt = {}
    if l2.type == "weighted_sum":
        z = (h * tp["v"]).sum(-1)
        g = dy * dact(z, l2.out_activation)
        dh = g[..., None] * tp["v"]
        dt["v"] = (g[..., None] * h).sum(0)
    else:
        pooled, dpool = _pool(h, l2)
        g = dy * dact(pooled, l2.out_activation)
        dh = g[..., None] * dpool
    tr = l1.transform
    if tr == "none":
        dF = dh
    elif tr == "activation":
        dF = dh * dact(F, l1.transform_activation)
    elif tr == "affine":
        du = dh * dact(u, l1.transform_activation)
        dF = du * tp["alpha"]
        dt["alpha"] = (du * F).sum(0)
        dt["beta"] = du.sum(0)
    else:  # gate: h = F sigmoid(u)
        sg = _sigmoid(u)
        du = dh * F * sg * (1.0 - sg)
        dF = dh * sg + du * tp["alpha"]
        dt["alpha"] = (du * F).sum(0)
        dt["beta"] = du.sum(0)
    return dF, dt


# ----------------------------------------------------------------------------- both levels


def forward_two_level(x, idx, w, bias, counts, gs: int, l1, l2, tparams):
    """(y [B, G], F [B, G, S], pre [B, G * S], mag [B, G * S]) float64."""
    G = len(counts)
    pre, mag, _ = level1_forward(x, idx, w, bias, counts, gs, l1.neurons_per_shard, l1)
    B = pre.shape[0]
    F = act(pre, l1.out_activation).reshape(B, G, -1)
    return level2_forward(F, l1, l2, tparams), F, pre, mag


def backward_two_level(x, idx, w, bias, counts, gs: int, l1, l2, tparams, dy):
    """(dW, db, dX, {name: d tparam}) float64 for upstream dy [B, G]."""
    _, F, pre, _ = forward_two_level(x, idx, w, bias, counts, gs, l1, l2, tparams)
    dF, dt = level2_backward(F, l1, l2, tparams, dy)
    B = pre.shape[0]
    g_pre = dF.reshape(B, -1) * dact(pre, l1.out_activation)
    dW, db, dX = level1_backward(x, idx, w, bias, counts, gs, l1.neurons_per_shard, l1, g_pre)
    return dW, db, dX, dt
