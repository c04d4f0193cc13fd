"""Custom autograd: forward saves no hidden activations; backward recomputes them.

Mirrors sparse_pooling/autograd.py for the level-1 path (the two-level function is in semantic.py):

* ``Level1Runtime`` (autograd.py:68-300): executes the fused kernels of one layer, holds no
  tensor of size [B, H], records ``last_info``;
* ``SparsePoolFunction`` (autograd.py:380-414): saves (x, W, b, pre), recomputes in backward,
  routes dW/db into fp32 ``main_grad`` buffers when present (autograd.py:357-363);
* ``fit_policy`` / ``resolve_policy`` / ``AUTO_POLICY`` (autograd.py:30-65).

The only executor is the HIP backend (granulelayer_amd.backend); there is no Triton or PyTorch
fallback, so a runtime on a CPU device refuses to run.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional

import torch

from .config import LevelSpec, PhysicalPlan, check_workspace_budget, resolve_reduction
from .layout import SparseLayout

AUTO_POLICY = {"max": "save_winners", "topk_mean": "save_winners", "mean": "minimal_stats",
               "logmeanexp": "minimal_stats", "power_mean": "minimal_stats", "softmax_weighted": "minimal_stats",
               "sum": "minimal_stats"}


def resolve_policy(level: LevelSpec, requested: str) -> str:
    if requested == "auto":
        return AUTO_POLICY[level.type]
    if requested == "save_winners" and level.type not in ("max", "topk_mean"):
        return "minimal_stats"  # no winners to save; the reference's documented fallback
    return requested


# bytes of saved selection ids (max winners, top-k slots) above which save_winners falls back to
# recomputing them in backward, and the id-tensor size per token chunk of that recomputation
# (the reference's CHECKPOINT_BUDGET / RECOMPUTE_CHUNK_BYTES, sparse_pooling/autograd.py:41-42)
CHECKPOINT_BUDGET = 2 << 30
RECOMPUTE_CHUNK_BYTES = 512 << 20


def _ids_per_token(rt: "Level1Runtime") -> int:
    """int32 selection ids one token keeps: U units x k (top-k mean) or x 1 (max); 0 otherwise."""
    lv = rt.level
    if lv.type not in ("max", "topk_mean"):
        return 0
    return rt.units.U * (lv.k if lv.type == "topk_mean" else 1)


def fit_policy(rt: "Level1Runtime", policy: str, batch: int) -> str:
    """save_winners keeps B x U x k int32 ids; above CHECKPOINT_BUDGET the backward recomputes them
    instead and ``last_info['policy_fallback']`` says so (sparse_pooling/autograd.py:45-56)."""
    if policy == "save_winners":
        need = batch * _ids_per_token(rt) * 4
        if need > CHECKPOINT_BUDGET:
            rt.last_info["policy_fallback"] = f"save_winners needs {need / 2**30:.1f} GiB of ids -> minimal_stats"
            return "minimal_stats"
    rt.last_info.pop("policy_fallback", None)
    return policy


def recompute_chunk(rt: "Level1Runtime") -> int:
    """Tokens per chunk when selection ids are recomputed in backward: the [b, U, k] id tensor of a
    chunk stays within RECOMPUTE_CHUNK_BYTES, at least 32 tokens, a multiple of 32
    (sparse_pooling/autograd.py:335)."""
    per = max(_ids_per_token(rt) * 4, 1)
    return max(32, (min(RECOMPUTE_CHUNK_BYTES, CHECKPOINT_BUDGET) // per) // 32 * 32)


def act_torch(x: torch.Tensor, name: str) -> torch.Tensor:
    """Out-activation of the pooled value (kernels/ops.py:165-170): identity, relu or exact (erf) gelu."""
    if name == "identity":
        return x
    if name == "relu":
        return torch.relu(x)
    if name == "gelu":
        return torch.nn.functional.gelu(x)
    raise NotImplementedError(f"out-activation {name!r}")


def dact_torch(x: torch.Tensor, name: str) -> torch.Tensor:
    """Derivative of act_torch (kernels/ops.py:173-179): gelu'(x) = Phi(x) + x phi(x)."""
    if name == "identity":
        return torch.ones_like(x)
    if name == "relu":
        return (x > 0).to(x.dtype)
    if name == "gelu":
        cdf = 0.5 * (1.0 + torch.erf(x * 0.7071067811865476))
        return cdf + x * 0.3989422804014327 * torch.exp(-0.5 * x * x)
    raise NotImplementedError(f"out-activation {name!r}")


@dataclass
class Units:
    """Level-1 pooling units (kernels/ops.py:30-56): one unit per group for a single level."""

    S: int
    BPS: int
    nps: Optional[int]
    counts: torch.Tensor

    @property
    def U(self) -> int:
        return self.counts.numel()


def make_units(layout: SparseLayout, nps: Optional[int], device) -> Units:
    """Pooling units (sparse_pooling/kernels/ops.py:45-56): the groups, or with neurons_per_shard
    nps the S = ceil(max_group / nps) shards of every group, unit u = g * S + s pooling slots
    [s * nps, s * nps + counts[u]) of group g.  Every shard must hold a neuron."""
    n_g = layout.counts_tensor(device).to(torch.float32)
    if nps is None:
        return Units(1, layout.blocks_per_group, None, n_g)
    if nps % (4 * layout.block) != 0:
        raise ValueError(f"neurons_per_shard must be a multiple of 4*C = {4 * layout.block}")
    S = -(-layout.max_group // nps)
    s = torch.arange(S, device=device, dtype=torch.float32)
    cnt = torch.clamp(n_g[:, None] - s[None, :] * nps, min=0, max=nps)
    if bool((cnt == 0).any()):
        raise ValueError("a semantic shard would be empty; choose a different neurons_per_shard")
    return Units(S, nps // layout.block, nps, cnt.reshape(-1))


class Level1Runtime:
    """Executes the fused level-1 kernels for one layer (sparse_pooling/autograd.py:68-300)."""

    def __init__(self, layout: SparseLayout, idx: torch.Tensor, level: LevelSpec, plan: PhysicalPlan,
                 nps: Optional[int] = None, workspace_budget: Optional[int] = None,
                 backend: Optional[object] = None):
        reason = level.hip_reason()
        if reason:
            raise NotImplementedError(reason)
        if layout.shared_indices and not getattr(layout, "rec_shift", 0):
            raise NotImplementedError("Mode B (block-shared indices) is not on the MI355X path")
        if nps is not None and getattr(layout, "rec_shift", 0):
            raise NotImplementedError("semantic two-level pooling over shared index records is not on the MI355X path")
        if plan.backend == "triton":
            raise NotImplementedError("backend='triton': the MI355X build has no Triton path (use 'hip')")
        self.layout = layout
        self.idx = idx
        self.level = level
        self.plan = plan
        self.counts_i32 = layout.counts_tensor(idx.device).contiguous()
        self.units = make_units(layout, nps, idx.device)
        # valid neurons per pooling unit (the groups, or the level-1 shards), as the kernels read them
        self.unit_counts_i32 = (self.counts_i32 if nps is None
                                else self.units.counts.to(torch.int32).contiguous())
        self.workspace_budget = check_workspace_budget(workspace_budget)
        if backend is None and idx.is_cuda:
            from .backend import backend_for

            backend = backend_for(idx.device)
        self.backend = backend
        self.last_info: Dict = {}
        self.det = False
        self.grad_call = True  # set per call by the layer: grad mode was on (a backward can follow)

    def check_devices(self, *tensors):
        dev = self.idx.device
        for t in tensors:
            if t is not None and t.device != dev:
                raise ValueError(f"tensor on {t.device} but the layer's parameters are on {dev} "
                                 "(move the input or the layer)")

    def _require_backend(self):
        if self.backend is None:
            raise RuntimeError(f"parameters on {self.idx.device}: the MI355X path runs on a ROCm GPU only "
                               "(no CPU / PyTorch fallback)")

    def resolve_reduction(self, B: int) -> bool:
        mode, why, _ = resolve_reduction(self.plan)
        self.det = mode == "deterministic"
        self.last_info["reduction"] = {"mode": mode, "reason": why}
        return self.det

    def describe_execution(self) -> Dict:
        out = {"backend": "hip"}
        if self.backend is not None:
            out["build"] = self.backend.build_info()
        return out

    # ---------------------------------------------------------------- forward
    def forward(self, x: torch.Tensor, w, b, track_ids: bool = False, relu_mask: bool = False) -> Dict[str, torch.Tensor]:
        """Merged statistics: {'pre': [B, U]} (the pooled value before the out-activation); with
        relu_mask, also the ReLU bits the HIP backward can use instead of recomputing z."""
        self.check_devices(x, w, b)
        self._require_backend()
        self.resolve_reduction(x.shape[0])
        out = (self.backend.forward(self, x, w, b, track_ids, relu_mask=True) if relu_mask
               else self.backend.forward(self, x, w, b, track_ids))
        self.last_info["forward_backend"] = "hip"
        self.last_info["forward_relu_mask"] = "relu_mask" in out
        return out

    # --------------------------------------------------------------- backward
    def backward(self, x, w, b, g_pre: torch.Tensor, saved: Dict[str, torch.Tensor], policy: str,
                 dw_buf: torch.Tensor, db_buf: torch.Tensor, recomputed: bool = False) -> torch.Tensor:
        """Accumulate dW/db into the fp32 buffers, return dX (fp32, [B, D])."""
        self.last_info["policy"] = policy
        self.check_devices(x, w, b, g_pre, dw_buf, db_buf)
        self._require_backend()
        self.resolve_reduction(x.shape[0])
        self.last_info["recomputed_stats"] = recomputed
        self.last_info["backward_backend"] = "hip"
        return self.backend.backward(self, x, w, b, g_pre, saved, dw_buf, db_buf)


def _compute_operands(x, w, b, compute_dtype):
    """Operands of the kernels (autograd.py:349-354).  The HIP kernels read x, W and b as fp32 or
    bf16 and compute in fp32 (bf16 values are widened in the kernel, as the reference's kernels
    widen W, triton_fused.py:257).  A bf16 compute dtype rounds x, W and b to bf16 as the
    reference's cast does; parameters already stored in bf16 (the reference's default layer dtype)
    are passed as they are, with no copy."""
    if compute_dtype == torch.bfloat16:
        xc = x.to(torch.bfloat16).contiguous()
        wc = w if w.dtype == torch.bfloat16 else w.to(torch.bfloat16)
        bc = b if b.dtype == torch.bfloat16 else b.to(torch.bfloat16)
    elif compute_dtype == torch.float32:
        xc = x if x.dtype in (torch.float32, torch.bfloat16) else x.to(torch.float32)
        xc = xc.contiguous()
        wc = w if w.dtype in (torch.float32, torch.bfloat16) else w.to(torch.float32)
        bc = b if b.dtype in (torch.float32, torch.bfloat16) else b.to(torch.float32)
    else:
        raise NotImplementedError(f"compute dtype {compute_dtype} (the MI355X path computes fp32 or bf16 operands)")
    return xc, wc.contiguous(), bc.contiguous()


def _grad_buffers(w, b):
    mg_w = getattr(w, "main_grad", None)
    mg_b = getattr(b, "main_grad", None)
    if mg_w is not None and mg_b is not None:
        return mg_w, mg_b, True
    return (torch.zeros(w.shape, device=w.device, dtype=torch.float32),
            torch.zeros(b.shape, device=b.device, dtype=torch.float32), False)


def _saved_stats(level: LevelSpec, out: Dict[str, torch.Tensor], policy: str) -> Dict[str, torch.Tensor]:
    """What the forward keeps for backward (autograd.py:366-377): pre, with save_winners the
    max-pooling winner ids or the top-k slots, and softmax-weighted pooling's L2."""
    if policy == "recompute_stats":
        return {}
    keep = {"pre": out["pre"]}
    if "relu_mask" in out:  # the forward's ReLU bits (1/32 of the hidden tensor): dW skips the recompute
        keep["relu_mask"] = out["relu_mask"]
    for key in ("winner", "topk_slot"):
        if policy == "save_winners" and key in out:
            keep[key] = out[key]
    if level.type == "softmax_weighted" and policy == "minimal_stats":
        keep["L2"] = out["L2"]  # its backward needs the log-normaliser (autograd.py:375-376)
    return keep


def _level1_backward(rt: Level1Runtime, xc, wc, bc, dy, saved: Dict[str, torch.Tensor], policy: str, dw_buf,
                     db_buf, recomputed: bool = False) -> torch.Tensor:
    """dX of the level-1 kernels for dy [B, U], the gradient of out_act(pre); dW / db accumulate
    into the buffers.  Statistics the backward needs and the policy did not keep are recomputed
    (autograd.py:246-258): max / top-k pooling need the selected slots, softmax-weighted the L2;
    when the whole batch's slots would exceed CHECKPOINT_BUDGET they are recomputed and consumed
    one token chunk at a time (autograd.py:255-259, 329-343)."""
    lv = rt.level
    need = {"max": "winner", "topk_mean": "topk_slot", "softmax_weighted": "L2"}.get(lv.type)
    B = xc.shape[0]
    if need is not None and need not in saved and B * _ids_per_token(rt) * 4 > CHECKPOINT_BUDGET:
        return _chunked_selection_backward(rt, xc, wc, bc, dy, saved.get("pre"), policy, dw_buf, db_buf)
    if "pre" not in saved or (need is not None and need not in saved):
        saved.update(rt.forward(xc, wc, bc, track_ids=True))
        recomputed = True
    g_pre = dy.float() * dact_torch(saved["pre"], lv.out_activation)
    return rt.backward(xc, wc, bc, g_pre.contiguous(), saved, policy, dw_buf, db_buf, recomputed)


def _chunked_selection_backward(rt: Level1Runtime, xc, wc, bc, dy, pre, policy, dw_buf, db_buf):
    """Max / top-k backward with the selection ids recomputed per token chunk, so the [b, U, k] id
    tensor of one chunk stays within RECOMPUTE_CHUNK_BYTES; dW / db accumulate over the chunks.
    The total extra work is one forward (sparse_pooling/autograd.py:329-343)."""
    B, D = xc.shape
    bc_tok = recompute_chunk(rt)
    dx = torch.empty((B, D), device=xc.device, dtype=torch.float32)
    for s0 in range(0, B, bc_tok):
        xs = xc[s0:s0 + bc_tok]
        st = rt.forward(xs, wc, bc, track_ids=True)
        p = st["pre"] if pre is None else pre[s0:s0 + bc_tok]
        g = (dy[s0:s0 + bc_tok].float() * dact_torch(p, rt.level.out_activation)).contiguous()
        dx[s0:s0 + bc_tok] = rt.backward(xs, wc, bc, g, st, policy, dw_buf, db_buf, True)
        del st
    rt.last_info["backward_token_chunks"] = -(-B // bc_tok)
    return dx


class SparsePoolFunction(torch.autograd.Function):
    """Single level: y [B, G] = out_act(pool(sparse_projection(x)))."""

    @staticmethod
    def forward(ctx, x, w, b, rt: Level1Runtime, policy: str, compute_dtype):
        policy = fit_policy(rt, policy, x.shape[0])
        xc, wc, bc = _compute_operands(x, w, b, compute_dtype)
        lv = rt.level
        # the ReLU bits (PhysicalPlan.relu_bits="keep") only when a backward can run (grad mode on
        # at the call, recorded by rt.grad_call: inside forward it is always off) and the policy
        # keeps statistics
        keep_bits = (getattr(rt.plan, "relu_bits", "recompute") == "keep" and policy != "recompute_stats"
                     and getattr(rt, "grad_call", True) and any(ctx.needs_input_grad[:3]))
        out = rt.forward(xc, wc, bc, track_ids=(policy == "save_winners"), relu_mask=keep_bits)
        pre = out["pre"]
        y = act_torch(pre, lv.out_activation)
        saved = _saved_stats(lv, out, policy)
        ctx.rt, ctx.policy, ctx.compute_dtype = rt, policy, compute_dtype
        ctx.saved_keys = list(saved.keys())
        ctx.save_for_backward(x, w, b, *saved.values())
        rt.last_info["checkpoint_bytes"] = sum(t.numel() * t.element_size() for t in saved.values())
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, b, *svals = ctx.saved_tensors
        saved = dict(zip(ctx.saved_keys, svals))
        rt: Level1Runtime = ctx.rt
        xc, wc, bc = _compute_operands(x, w, b, ctx.compute_dtype)
        dw_buf, db_buf, use_main = _grad_buffers(w, b)
        dx = _level1_backward(rt, xc, wc, bc, dy, saved, ctx.policy, dw_buf, db_buf)
        gw = None if use_main else dw_buf.to(w.dtype)
        gb = None if use_main else db_buf.to(b.dtype)
        return dx.to(x.dtype, memory_format=torch.contiguous_format), gw, gb, None, None, None


# the two-level function lives beside its level-2 code; exported here as the reference's module does
from .semantic import SemanticPoolFunction  # noqa: E402,F401
