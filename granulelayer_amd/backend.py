"""HIP backend object: the drop-in boundary of the reference's native backend.

``HipBackend`` exposes the two methods the reference's ``Level1Runtime`` calls on its native
backend (sparse_pooling/autograd.py:220-223 and :265-267; implemented for CUDA at
sparse_pooling/backends/cuda/runtime.py:339-712):

    forward(rt, x, w, b, track_ids)                     -> {"pre": [B, U] fp32[, "winner" | "topk_slot"]}
    backward(rt, x, w, b, g_pre, stats, dw_buf, db_buf) -> dX [B, D] fp32 (dW/db accumulated)

plus ``adam`` (the FusedAdamW launch, sparse_pooling/optim.py:116-123) and ``edges`` (the
input-major edge list the deterministic dX kernel consumes, built once per index tensor).

Every launch runs under ``torch.cuda.device(<tensor device>)`` on that device's current stream,
asynchronously; buffers (outputs and workspace) are allocated by PyTorch and passed as raw
pointers.  Any refusal of the native library raises ``NativeError``; there is no fallback.
"""
from __future__ import annotations

import ctypes
import threading
from typing import Dict, Optional

import numpy as np
import torch

from . import _native as N

# Default dz budget of the smooth pools' backward: 64 GiB of MI355X's 288 GB HBM.  100.6 M neurons
# (C2) then run 128-token chunks instead of the library default's 64, and the recompute and dense
# dX passes cost less per token in longer chunks.
DZ_BUDGET = 64 * 2**30

# The forward's ReLU bits kept for the backward (GlFwdArgs.relu_mask): one bit per (token, neuron),
# 1/32 of the [B, N] hidden tensor's fp32 bytes (3.2 GB at C2, 12.9 GB at C4).  With them the
# backward's dW pass does not recompute z.  Kept only up to this size; larger layers recompute.
RELU_MASK_BUDGET = 16 * 2**30


def _ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.data_ptr()


def _stream(dev) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _x_operand(x: torch.Tensor):
    """(tensor, dtype code, row stride) of the input: fp32 or bf16, unit feature stride."""
    if x.dim() != 2:
        raise ValueError(f"x must be [B, D] (got {tuple(x.shape)})")
    if x.dtype == torch.float32:
        code = N.GL_DTYPE_F32
    elif x.dtype == torch.bfloat16:
        code = N.GL_DTYPE_BF16
    else:
        raise TypeError(f"x must be float32 or bfloat16 (got {x.dtype})")
    if x.stride(1) != 1 or x.stride(0) < x.shape[1]:
        x = x.contiguous()
    return x, code, x.stride(0)


def _params(w: torch.Tensor, b: torch.Tensor):
    """(W, bias, dtype code) as the kernels read them: fp32 or bf16 (widened in the kernels), both
    of one dtype (a bf16 / fp32 mix is widened to fp32, exactly), contiguous, W 4-byte aligned."""
    for name, t in (("weight", w), ("bias", b)):
        if t.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"{name} must be float32 or bfloat16 (got {t.dtype})")
    if w.dtype != b.dtype:
        w, b = w.float(), b.float()
    w, b = w.contiguous(), b.contiguous()
    if w.data_ptr() % 4:  # a bf16 view at an odd element offset: the dX kernels read 32-bit words
        w = w.clone()
    return w, b, N.GL_DTYPE_BF16 if w.dtype == torch.bfloat16 else N.GL_DTYPE_F32


def _f32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32 (got {t.dtype})")
    return t.contiguous()


class HipBackend:
    """The MI355X HIP backend (one per process; the library is device-independent)."""

    _instance = None
    _lock = threading.Lock()

    def __init__(self, lib: Optional[N.Library] = None, window_staging: bool = True):
        self.lib = lib or N.library()
        # stage only each pool's input window in LDS when the windows are narrow (same results)
        self.window_staging = window_staging

    @classmethod
    def get(cls) -> "HipBackend":
        with cls._lock:
            if cls._instance is None:
                cls._instance = cls()
            return cls._instance

    def build_info(self) -> Dict:
        return {"library": str(self.lib.path), "abi_version": N.ABI_VERSION, "arch": "gfx950"}

    # ------------------------------------------------------------------ helpers
    @staticmethod
    def _layer(rt):
        L = rt.layout
        G, S, K = L.groups, L.slots_per_group, L.fan_in
        return L, G, S, K

    @staticmethod
    def _pools(rt):
        """Pool geometry of the launches: (pools U, slots per pool, shards per group sps, group
        stride gs, valid neurons per pool [U] int32).  A single level pools the groups; a two-level
        layer's level 1 pools the S shards of nps slots of every group (unit u = g * S + s,
        sparse_pooling/kernels/ops.py:30-56)."""
        L = rt.layout
        u = getattr(rt, "units", None)
        counts = getattr(rt, "unit_counts_i32", rt.counts_i32)
        if u is None or u.nps is None or u.S == 1:
            # one unit per group (a single shard spans its whole group): the groups' own geometry
            geo = (L.groups, L.slots_per_group, 1, L.slots_per_group, counts)
        else:
            geo = (L.groups * u.S, u.nps, u.S, L.slots_per_group, counts)
        U, S, sps, gs, _ = geo
        rows = U * S if sps == 1 else U // sps * gs
        if rows != L.groups * L.slots_per_group or counts.numel() != U:
            raise RuntimeError(f"pool geometry (U={U}, S={S}, sps={sps}, gs={gs}) does not address the layout's "
                               f"{L.groups * L.slots_per_group} slots")
        return geo

    @staticmethod
    def rec_shift(rt) -> int:
        """log2 slots per shared index record: 0 for Mode A, 4 for the K16 / C16 records of
        Cover-TopK/16 (granulelayer_amd.cover_topk16.CompactLayout)."""
        return int(getattr(rt.layout, "rec_shift", 0))

    @staticmethod
    def _codes(rt):
        lv = rt.level
        reason = lv.hip_reason()
        if reason:
            raise NotImplementedError(reason)
        return N.GL_ACT[lv.activation], N.GL_POOL[lv.type]

    @staticmethod
    def _check(rt, x, w, b):
        L = rt.layout
        dev = rt.idx.device
        for name, t in (("x", x), ("weight", w), ("bias", b)):
            if t.device != dev:
                raise ValueError(f"{name} on {t.device} but the layer's parameters are on {dev}")
        if not dev.type == "cuda":
            raise RuntimeError("the HIP backend needs the layer on a ROCm GPU (no CPU path)")
        if x.shape[-1] != L.input_dim:
            raise ValueError(f"x has {x.shape[-1]} features, layer expects {L.input_dim}")
        if tuple(w.shape) != tuple(L.weight_shape) or tuple(b.shape) != tuple(L.bias_shape):
            raise ValueError("weight / bias shapes do not match the layout")

    # ------------------------------------------------------------------ forward
    def forward(self, rt, x, w, b, track_ids: bool = False, relu_mask: bool = False) -> Dict[str, torch.Tensor]:
        """The reference's backend forward (sparse_pooling/autograd.py:220-223).  relu_mask: also
        return the ReLU bits of every (token, neuron) as "relu_mask" when the layer has them
        (ReLU sum / mean at fan-in 8) and they fit RELU_MASK_BUDGET, for the backward."""
        self._check(rt, x, w, b)
        L, _, _, K = self._layer(rt)
        G, S, sps, gs, counts = self._pools(rt)
        act, pool = self._codes(rt)
        x, xcode, sxb = _x_operand(x)
        w, b, wcode = _params(w, b)
        B = x.shape[0]
        pre = torch.empty((B, G), device=x.device, dtype=torch.float32)
        # with track_ids, the selected slots: max pooling's "winner" [B, U] and top-k mean's
        # "topk_slot" [B, U, k] (best first, -1 past min(n_g, k)), the reference's statistics
        # (kernels/ops.py:189-195, 212-228)
        topk = rt.level.k if pool == N.GL_POOL["topk_mean"] else 0
        winner, key = None, None
        if track_ids and pool == N.GL_POOL["max"]:
            winner, key = torch.empty((B, G), device=x.device, dtype=torch.int32), "winner"
        elif track_ids and topk:
            winner, key = torch.empty((B, G, topk), device=x.device, dtype=torch.int32), "topk_slot"
        out = {"pre": pre} if winner is None else {"pre": pre, key: winner}
        # LogMeanExp / softmax-weighted: the base-2 log-normaliser, the reference's "L2" statistic
        # (kernels/ops.py:201-209)
        lse = None
        if rt.level.type in ("logmeanexp", "softmax_weighted"):
            lse = torch.empty((B, G), device=x.device, dtype=torch.float32)
            out["L2"] = lse
        if B == 0:
            return out
        win_lo, win_width = self.windows(rt)
        a = N.GlFwdArgs(X=_ptr(x), sxb=sxb, x_dtype=xcode, B=B, D=L.input_dim, G=G, S=S, K=K, act=act, pool=pool,
                        topk=topk, rec_shift=self.rec_shift(rt), sps=sps, gs=gs, idx=_ptr(rt.idx), W=_ptr(w), bias=_ptr(b),
                        counts=_ptr(counts),
                        sched=_ptr(self.schedule(rt)), win=_ptr(win_lo), win_width=win_width, pre=_ptr(pre),
                        winner=_ptr(winner), pool_param=self.pool_param(rt), lse=_ptr(lse),
                        part_budget=self.part_budget(rt), w_dtype=wcode)
        with torch.cuda.device(x.device):
            if relu_mask:
                mb = self.lib.size_query("gl_fwd_mask_bytes", a)
                if 0 < mb <= RELU_MASK_BUDGET:
                    out["relu_mask"] = torch.empty(mb, device=x.device, dtype=torch.uint8)
                    a.relu_mask = _ptr(out["relu_mask"])
            need = self.lib.size_query("gl_fwd_workspace", a)
            ws = torch.empty(max(need, 1), device=x.device, dtype=torch.uint8)
            a.ws, a.ws_bytes = _ptr(ws), need
            self.lib.call("gl_fwd", ctypes.byref(a), ctypes.c_void_p(_stream(x.device)))
        rt.last_info["workspace_bytes"] = need
        return out

    @staticmethod
    def pool_param(rt) -> float:
        """The smooth operators' parameter: temperature (LogMeanExp), p (power mean), beta
        (softmax-weighted); 0 otherwise."""
        lv = rt.level
        return {"logmeanexp": lv.temperature, "power_mean": lv.p, "softmax_weighted": lv.beta}.get(lv.type, 0.0)

    @staticmethod
    def part_budget(rt) -> int:
        """Bytes of per-chunk forward partials one pass may hold: the layer's ``workspace_budget``
        when the caller set one (any value, the reference's 512 MiB default included), else 0 (the
        library's default of 8 GiB, which runs the BASELINE shapes' sum / mean forward in one
        pass).  The forward runs token chunks within it."""
        wb = getattr(rt, "workspace_budget", None)
        return 0 if wb is None else int(wb)

    @staticmethod
    def dz_budget(rt) -> int:
        """Bytes of per-neuron dz one backward token chunk of a smooth pool (LogMeanExp, power mean,
        softmax-weighted) may hold: the layer's ``workspace_budget`` when the caller set one, else
        DZ_BUDGET.  A fixed figure, not one taken from the free memory, because the chunking sets
        the order in which dW and db sum over the tokens."""
        wb = getattr(rt, "workspace_budget", None)
        return DZ_BUDGET if wb is None else int(wb)

    # ------------------------------------------------------------------ gather schedule
    def schedule(self, rt) -> Optional[torch.Tensor]:
        """Gather schedule of rt's index tensor for the forward / dW kernels (fan-in 8, one index
        record per slot), built on the GPU once per index tensor (gl_sched_build, the host
        builder's algorithm) and cached on rt; None otherwise."""
        L, _, _, K = self._layer(rt)
        G, S, sps, gs, counts = self._pools(rt)
        if K != 8 or self.rec_shift(rt):
            return None
        key = (rt.idx.data_ptr(), rt.idx._version)
        cached = getattr(rt, "_hip_sched", None)
        if cached is not None and cached[0] == key:
            return cached[1]
        dev = rt.idx.device
        n = ctypes.c_size_t(0)
        self.lib.call("gl_sched_size", G, S, K, ctypes.byref(n))
        sched = torch.empty(n.value // 4, dtype=torch.int32, device=dev)
        with torch.cuda.device(dev):
            self.lib.call("gl_sched_build", _ptr(rt.idx), _ptr(counts), L.input_dim, G, S, sps, gs, K, _ptr(sched),
                          ctypes.c_void_p(_stream(dev)))
        rt._hip_sched = (key, sched)
        return sched

    # ------------------------------------------------------------------ pool windows
    def windows(self, rt):
        """Per-pool input windows of rt's index tensor (first input per pool on the device, widest
        width), built on the GPU once per index tensor (gl_window_build) and cached on rt; (None, 0)
        when ``window_staging`` is off.  The library stages only the windows when they are narrow."""
        if not self.window_staging:
            return None, 0
        L, _, _, K = self._layer(rt)
        G, S, sps, gs, counts = self._pools(rt)
        key = (rt.idx.data_ptr(), rt.idx._version)
        cached = getattr(rt, "_hip_win", None)
        if cached is not None and cached[0] == key:
            return cached[1]
        dev = rt.idx.device
        lo = torch.empty(G, dtype=torch.int32, device=dev)
        width = torch.empty(1, dtype=torch.int32, device=dev)
        with torch.cuda.device(dev):
            self.lib.call("gl_window_build", _ptr(rt.idx), _ptr(counts), L.input_dim, G, S, sps, gs, K,
                          self.rec_shift(rt), _ptr(lo), _ptr(width), ctypes.c_void_p(_stream(dev)))
        out = (lo, int(width.item()))  # the launch needs the width on the host: one 4-byte copy
        rt._hip_win = (key, out)
        return out

    # ------------------------------------------------------------------ edges
    def edges(self, rt) -> torch.Tensor:
        """Input-major edge structure of rt's index tensor (built once, cached on rt)."""
        key = (rt.idx.data_ptr(), rt.idx._version)
        cached = getattr(rt, "_hip_edges", None)
        if cached is not None and cached[0] == key:
            return cached[1]
        L, _, _, K = self._layer(rt)
        G, S, sps, gs, counts = self._pools(rt)
        a = N.GlEdgeArgs(idx=_ptr(rt.idx), counts=_ptr(counts), D=L.input_dim, G=G, S=S, K=K,
                         rec_shift=self.rec_shift(rt), sps=sps, gs=gs)
        dev = rt.idx.device
        with torch.cuda.device(dev):
            eb, wb = self.lib.edges_size(a)
            edges = torch.empty(eb, device=dev, dtype=torch.uint8)
            ws = torch.empty(max(wb, 1), device=dev, dtype=torch.uint8)
            a.edges, a.edges_bytes, a.ws, a.ws_bytes = _ptr(edges), eb, _ptr(ws), wb
            self.lib.call("gl_edges_build", ctypes.byref(a), ctypes.c_void_p(_stream(dev)))
        # the scratch returns to PyTorch's stream-ordered cache: later allocations on this stream
        # are ordered after the build
        rt._hip_edges = (key, edges)
        return edges

    # ------------------------------------------------------------------ backward
    def backward(self, rt, x, w, b, g_pre, stats, dw_buf, db_buf) -> torch.Tensor:
        self._check(rt, x, w, b)
        L, _, _, K = self._layer(rt)
        G, S, sps, gs, counts = self._pools(rt)
        act, pool = self._codes(rt)
        x, xcode, sxb = _x_operand(x)
        w, b, wcode = _params(w, b)
        g_pre = _f32(g_pre, "g_pre")
        B, D = x.shape
        if tuple(g_pre.shape) != (B, G):
            raise ValueError(f"g_pre must be [{B}, {G}] (got {tuple(g_pre.shape)})")
        for name, t, shape in (("dw_buf", dw_buf, L.weight_shape), ("db_buf", db_buf, L.bias_shape)):
            if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != tuple(shape):
                raise ValueError(f"{name} must be a contiguous float32 tensor of shape {tuple(shape)}")
        # max / top-k mean: the selected neurons are the only ones with a gradient
        winner, topk = None, 0
        if pool in (N.GL_POOL["max"], N.GL_POOL["topk_mean"]):
            key, shape = ("winner", (B, G)) if pool == N.GL_POOL["max"] else ("topk_slot", (B, G, rt.level.k))
            topk = rt.level.k if pool == N.GL_POOL["topk_mean"] else 0
            winner = stats.get(key)
            if winner is None:
                raise ValueError(f"{rt.level.type} backward needs the forward's selected slots (stats[{key!r}])")
            if winner.dtype != torch.int32 or tuple(winner.shape) != shape or winner.device != x.device:
                raise ValueError(f"{key} must be an int32 {list(shape)} tensor on {x.device}")
            winner = winner.contiguous()
        # smooth pools: the forward's pooled values and L2 give the backward's coefficients
        pre, lse = None, None
        if rt.level.type in ("logmeanexp", "power_mean", "softmax_weighted"):
            pre = stats.get("pre")
            lse = stats.get("L2")
            if pre is None or (rt.level.type == "softmax_weighted" and lse is None):
                raise ValueError(f"{rt.level.type} backward needs the forward's statistics (pre and L2)")
            pre = _f32(pre, "pre")
            lse = None if lse is None else _f32(lse, "L2")
        dx = torch.empty((B, D), device=x.device, dtype=torch.float32)
        if B == 0:
            return dx
        win_lo, win_width = self.windows(rt)
        edges = self.edges(rt)
        a = N.GlBwdArgs(X=_ptr(x), sxb=sxb, x_dtype=xcode, B=B, D=D, G=G, S=S, K=K, act=act, pool=pool,
                        topk=topk, rec_shift=self.rec_shift(rt), sps=sps, gs=gs, idx=_ptr(rt.idx), W=_ptr(w), bias=_ptr(b),
                        counts=_ptr(counts),
                        sched=_ptr(self.schedule(rt)), win=_ptr(win_lo), win_width=win_width, g_pre=_ptr(g_pre),
                        winner=_ptr(winner), pool_param=self.pool_param(rt), pre=_ptr(pre), lse=_ptr(lse),
                        dW=_ptr(dw_buf), db=_ptr(db_buf), dX=_ptr(dx), edges=_ptr(edges),
                        edges_bytes=edges.numel(), dz_budget=self.dz_budget(rt), w_dtype=wcode)
        # the forward's ReLU bits, when it kept them: the dW pass then skips the recompute of z
        rm = stats.get("relu_mask")
        if rm is not None:
            fa = N.GlFwdArgs(B=B, D=D, G=G, S=S, K=K, act=act, pool=pool, rec_shift=self.rec_shift(rt), x_dtype=xcode)
            want = self.lib.size_query("gl_fwd_mask_bytes", fa)
            if rm.dtype != torch.uint8 or rm.numel() != want or want == 0 or rm.device != x.device:
                raise ValueError("relu_mask does not come from this layer's forward of this batch")
            a.relu_mask = _ptr(rm)
        rt.last_info["backward_relu_mask"] = rm is not None
        with torch.cuda.device(x.device):
            need = self.lib.size_query("gl_bwd_workspace", a)
            ws = torch.empty(max(need, 1), device=x.device, dtype=torch.uint8)
            a.ws, a.ws_bytes = _ptr(ws), need
            self.lib.call("gl_bwd", ctypes.byref(a), ctypes.c_void_p(_stream(x.device)))
        rt.last_info["backward_workspace_bytes"] = need
        return dx

    # ------------------------------------------------------------------ optimizer
    def adam(self, p, g, m, v, lr, beta1, beta2, eps, weight_decay, bc1, bc2, master=None, stochastic=False, seed=0):
        """In-place fused AdamW: p fp32 or bf16, g fp32 (zeroed), m/v fp32 or bf16.  bf16 p: with an
        fp32 ``master`` copy the update runs on it and p gets its nearest-even rounding; otherwise
        p is rounded stochastically (``stochastic``, Philox noise of ``seed``) or to nearest even
        (sparse_pooling/optim.py:26-64)."""
        if p.dtype not in (torch.float32, torch.bfloat16) or not p.is_contiguous():
            raise TypeError("param must be a contiguous float32 or bfloat16 tensor")
        if g.dtype != torch.float32 or not g.is_contiguous():
            raise TypeError("grad must be a contiguous float32 tensor")
        if m.dtype != v.dtype or m.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError("moments must both be float32 or bfloat16")
        if not (p.numel() == g.numel() == m.numel() == v.numel()):
            raise ValueError("param, grad and moments must have the same number of elements")
        if master is not None and (p.dtype != torch.bfloat16 or master.dtype != torch.float32
                                   or not master.is_contiguous() or master.numel() != p.numel()):
            raise ValueError("master must be a contiguous float32 copy of a bfloat16 parameter")
        bf = p.dtype == torch.bfloat16
        a = N.GlAdamArgs(p=_ptr(p), g=_ptr(g), m=_ptr(m), v=_ptr(v), n=p.numel(),
                         moments_dtype=N.GL_DTYPE_F32 if m.dtype == torch.float32 else N.GL_DTYPE_BF16,
                         lr=lr, beta1=beta1, beta2=beta2, eps=eps, weight_decay=weight_decay, bc1=bc1, bc2=bc2,
                         p_dtype=N.GL_DTYPE_BF16 if bf else N.GL_DTYPE_F32,
                         stochastic=int(bf and master is None and stochastic), master=_ptr(master),
                         seed=int(seed) & (2**64 - 1))
        with torch.cuda.device(p.device):
            self.lib.call("gl_adam", ctypes.byref(a), ctypes.c_void_p(_stream(p.device)))


def backend_for(device) -> HipBackend:
    """Backend of a device (the reference's backends.cuda.runtime.backend_for, runtime.py:188-197)."""
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError(f"no HIP backend for {dev}: the MI355X path needs a ROCm GPU")
    return HipBackend.get()
