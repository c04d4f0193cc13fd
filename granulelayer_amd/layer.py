"""PyTorch-facing module, mirroring sparse_pooling/layer.py (SparsePoolingLayer, layer.py:16-205).

Same constructor signature, buffers/parameters (``indices``, ``weight``, ``bias``), ``forward``,
``enable_main_grad`` / ``zero_main_grad``, ``last_info``, ``explain`` and ``effective_policy``.
On the MI355X path the layer runs the reference's Mode A (``shared_neurons=None``: every
neuron owns its own fan-in record) with every level-1 operator (mean, sum, max, top-k mean,
LogMeanExp, power mean, softmax-weighted; relu or identity neuron activations) and the semantic
two-level hierarchies (level-1 shards on the HIP kernels, level 2 in PyTorch, with the learned
transform / weighted-sum parameters ``t_alpha``, ``t_beta``, ``t_v`` of layer.py:89-100); other
configurations raise NotImplementedError naming what is unsupported.
"""
from __future__ import annotations

from typing import Optional, Union

import torch
from torch import nn

from .autograd import Level1Runtime, SparsePoolFunction, resolve_policy
from .semantic import SemanticPoolFunction
from .config import PhysicalPlan, PoolingConfig, check_workspace_budget
from .layout import SparseLayout, check_indices, init_parameters


class SparsePoolingLayer(nn.Module):
    """Weight-sparse projection to ``hidden_dim`` neurons (fan-in 8 or 16) fused with pooling to
    ``output_dim`` groups.  ``shared_neurons`` must be None (independent index records)."""

    def __init__(
        self,
        input_dim: int = 1024,
        hidden_dim: int = 100_000_000,
        output_dim: int = 1024,
        fan_in: int = 8,
        shared_neurons: Optional[int] = 8,
        pooling: Union[str, dict, PoolingConfig] = "max",
        checkpoint_policy: str = "auto",
        dtype: torch.dtype = torch.bfloat16,
        plan: Optional[PhysicalPlan] = None,
        workspace_budget: Optional[int] = None,
        device=None,
        seed: int = 0,
        bias_std: float = 0.0,
        backend: str = "auto",
        weight_layout: str = "auto",
        connectivity=None,
    ):
        super().__init__()
        if shared_neurons is not None:
            raise NotImplementedError("shared_neurons (Mode B, block-shared index records) is not on the MI355X "
                                      "path; use shared_neurons=None")
        if connectivity is not None:
            raise NotImplementedError("input-supergroup connectivity is not on the MI355X path yet")
        if weight_layout not in ("auto", "canonical"):
            raise ValueError("weight_layout must be 'auto' or 'canonical' (packed storage is Mode B only)")
        if backend not in ("auto", "cuda", "hip"):
            raise ValueError("backend must be 'auto', 'cuda' or 'hip' (there is no Triton path)")
        self.cfg = PoolingConfig.parse(pooling, checkpoint_policy)
        if isinstance(pooling, (str, PoolingConfig)) or "checkpoint_policy" not in (pooling or {}):
            self.cfg.checkpoint_policy = checkpoint_policy
        reason = self.cfg.levels[0].hip_reason()
        if reason:
            raise NotImplementedError(reason)
        self.layout = SparseLayout(input_dim, hidden_dim, output_dim, fan_in, 8, False)
        self.compute_dtype = dtype
        self.plan = plan or PhysicalPlan()
        self.backend_name = backend
        # None: the library's own defaults (8 GiB of forward partials, 64 GiB of smooth-pool dz);
        # any explicit value, the reference's 512 MiB default included, bounds both workspaces
        self.workspace_budget = check_workspace_budget(workspace_budget)
        self.connectivity = None
        idx, w, b = init_parameters(self.layout, device or "cpu", dtype=dtype, seed=seed, bias_std=bias_std)
        self.register_buffer("indices", idx)
        self.weight = nn.Parameter(w)
        self.bias = nn.Parameter(b)
        self._tnames = []
        if self.cfg.is_semantic_hierarchy:
            # level-2 parameters per (group, shard), initialised as the reference does (layer.py:89-100)
            l1, l2 = self.cfg.levels
            S = -(-self.layout.max_group // l1.neurons_per_shard)
            self.num_shards = S
            G = output_dim
            if l1.transform in ("affine", "gate"):
                self.t_alpha = nn.Parameter(torch.ones(G, S, device=device))
                self.t_beta = nn.Parameter(torch.zeros(G, S, device=device))
                self._tnames += ["alpha", "beta"]
            if l2.type == "weighted_sum":
                self.t_v = nn.Parameter(torch.full((G, S), 1.0 / S, device=device))
                self._tnames += ["v"]
        self._rt = None
        self._rt_key = None

    # ------------------------------------------------------------------
    def _runtime(self) -> Level1Runtime:
        key = (self.indices.device, self.indices.data_ptr(), self.indices._version, id(self.plan))
        if self._rt is None or self._rt_key != key:
            check_indices(self.layout, self.indices)
            l1 = self.cfg.levels[0]
            self._rt = Level1Runtime(self.layout, self.indices, l1, self.plan,
                                     l1.neurons_per_shard if self.cfg.is_semantic_hierarchy else None,
                                     self.workspace_budget, None)
            self._rt_key = key
        return self._rt

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        # a checkpoint of an input-supergroup layer carries its plan as `sg_plan` (layer.py:133-142);
        # this layer has no connectivity, so such a checkpoint is refused as the reference refuses it
        if prefix + "sg_plan" in state_dict:
            raise ValueError("checkpoint and layer disagree on input-supergroup connectivity")
        key = prefix + "indices"
        if key in state_dict and state_dict[key].dtype == torch.int16:  # reference checkpoint
            state_dict[key] = state_dict[key].to(torch.int32)
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)
        self._rt = None

    @property
    def last_info(self):
        return {} if self._rt is None else dict(self._rt.last_info)

    def explain(self, batch: int = 8192) -> dict:
        """The execution the layer would use for ``batch`` tokens, without running it."""
        out = dict(backend_requested=self.backend_name)
        if not self.indices.is_cuda:
            out["backend"] = "none (CPU parameters)"
            return out
        rt = self._runtime()
        out.update(rt.describe_execution(), forward={"backend": "hip", "kernel": "fwd_kernel (neuron-stationary)"},
                   backward={"backend": "hip", "kernels": ["bwd_w_kernel", "dx_kernel or dx_dma_kernel", "dx_reduce_kernel"]},
                   batch=batch)
        return out

    @property
    def effective_policy(self) -> str:
        return resolve_policy(self.cfg.levels[0], self.cfg.checkpoint_policy)

    def enable_main_grad(self):
        """Accumulate W/b gradients into persistent fp32 ``main_grad`` buffers (autograd then
        returns None for them)."""
        for p in (self.weight, self.bias):
            if getattr(p, "main_grad", None) is None:
                p.main_grad = torch.zeros(p.shape, device=p.device, dtype=torch.float32)

    def zero_main_grad(self):
        for p in (self.weight, self.bias):
            if getattr(p, "main_grad", None) is not None:
                p.main_grad.zero_()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1])
        rt = self._runtime()
        if self.cfg.is_semantic_hierarchy:
            tparams = [getattr(self, "t_" + n) for n in self._tnames]
            y = SemanticPoolFunction.apply(x2, self.weight, self.bias, rt, self.cfg, self.effective_policy,
                                           self.compute_dtype, self._tnames, *tparams)
        else:
            rt.grad_call = torch.is_grad_enabled()
            y = SparsePoolFunction.apply(x2, self.weight, self.bias, rt, self.effective_policy, self.compute_dtype)
        return y.reshape(*lead, y.shape[-1])

    def extra_repr(self) -> str:
        L = self.layout
        return (f"in={L.input_dim}, hidden={L.hidden_dim:,}, out={L.groups}, fan_in={L.fan_in}, "
                f"mode=A(independent), pooling={self.cfg.describe()}, policy={self.effective_policy}")
