"""Configuration objects, mirroring the reference's public configuration API.

``LevelSpec`` / ``PoolingConfig`` / ``PhysicalPlan`` keep the reference's names, fields, defaults
and validation (sparse_pooling/config.py:22-224, 240-421) so existing call sites construct
them unchanged.  The MI355X path executes every level-1 operator of the reference -- Mean,
``"sum"`` (Mean x n_g, BASELINE's "sum pooling"), Max, Top-K mean, LogMeanExp, power mean and
softmax-weighted -- with identity, ReLU or exact (erf) GELU neuron activations (power mean: ReLU,
as the reference defines it), and the semantic two-level hierarchies (level 1 on the HIP kernels,
level 2 in PyTorch).  What it does not run (Mode B block-shared records, input-supergroup
connectivity) parses exactly as in the reference and is refused at run time with a clear error.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Union

POOL_TYPES = ("max", "topk_mean", "mean", "logmeanexp", "power_mean", "softmax_weighted", "sum")
LEVEL2_ONLY_TYPES = ("weighted_sum",)
ACTIVATIONS = ("identity", "relu", "gelu")
TRANSFORMS = ("none", "activation", "affine", "gate")
CHECKPOINT_POLICIES = ("minimal_stats", "recompute_stats", "save_winners", "auto")
POOL_ID = {name: i for i, name in enumerate(POOL_TYPES)}
ACT_ID = {name: i for i, name in enumerate(ACTIVATIONS)}

# operators executed by the HIP path (everything else parses but is refused at run time)
HIP_POOLS = ("mean", "sum", "max", "topk_mean", "logmeanexp", "power_mean", "softmax_weighted")
HIP_ACTIVATIONS = ("identity", "relu", "gelu")

_DEFAULT_ACT = {"max": "identity", "topk_mean": "identity", "mean": "relu", "logmeanexp": "identity",
                "power_mean": "relu", "softmax_weighted": "identity", "sum": "relu"}
_DEFAULT_OUT_ACT = {"max": "relu"}
_ALIASES = {"mean_relu": ("mean", {"activation": "relu"}), "lme": ("logmeanexp", {}),
            "softmax": ("softmax_weighted", {}), "power": ("power_mean", {}), "topk": ("topk_mean", {}),
            "sum_relu": ("sum", {"activation": "relu"})}


@dataclass
class LevelSpec:
    """One pooling level (fields and checks of sparse_pooling/config.py:69-161)."""

    type: str
    activation: str = ""
    out_activation: str = ""
    k: int = 8
    temperature: float = 1.0
    beta: float = 1.0
    p: float = 2.0
    neurons_per_shard: Optional[int] = None
    transform: str = "none"
    transform_activation: str = "relu"

    def __post_init__(self):
        if self.type in _ALIASES:
            t, extra = _ALIASES[self.type]
            self.type = t
            for k_, v in extra.items():
                if not getattr(self, k_):
                    setattr(self, k_, v)
        if self.type not in POOL_TYPES + LEVEL2_ONLY_TYPES:
            raise ValueError(f"unknown pooling type {self.type!r}")
        if not self.activation:
            self.activation = _DEFAULT_ACT.get(self.type, "identity")
        if not self.out_activation:
            self.out_activation = _DEFAULT_OUT_ACT.get(self.type, "identity")
        for a in (self.activation, self.out_activation):
            if a not in ACTIVATIONS:
                raise ValueError(f"unknown activation {a!r}")
        if self.transform not in TRANSFORMS:
            raise ValueError(f"unknown transform {self.transform!r}")
        if self.type == "topk_mean" and (self.k < 1 or (self.k & (self.k - 1)) != 0 or self.k > 64):
            raise ValueError("topk_mean k must be a power of two in [1, 64]")
        if self.type == "logmeanexp" and not self.temperature > 0:
            raise ValueError("temperature must be > 0")
        if self.type == "softmax_weighted" and not self.beta > 0:
            raise ValueError("beta must be > 0")
        if self.type == "power_mean" and not self.p >= 1:
            raise ValueError("power_mean requires p >= 1")
        if self.type == "power_mean" and self.activation != "relu":
            raise ValueError("power_mean is defined on relu activations")

    @property
    def pool_id(self) -> int:
        return POOL_ID[self.type]

    @property
    def act_id(self) -> int:
        return ACT_ID[self.activation]

    @property
    def out_act_id(self) -> int:
        return ACT_ID[self.out_activation]

    def hip_reason(self) -> str:
        """Why the HIP path cannot execute this level ("" if it can)."""
        if self.type not in HIP_POOLS:
            return f"pooling {self.type!r} is not on the MI355X path (supported: {', '.join(HIP_POOLS)})"
        if self.activation not in HIP_ACTIVATIONS:
            return f"activation {self.activation!r} is not on the MI355X path (supported: {', '.join(HIP_ACTIVATIONS)})"
        # out_activation is applied to pre by the autograd layer (torch): identity, relu and gelu
        if self.neurons_per_shard is not None and self.neurons_per_shard % 32 != 0:
            return "neurons_per_shard must be a multiple of 4*C = 32"
        return ""

    def describe(self) -> str:
        s = self.type
        if self.type == "topk_mean":
            s += f"(k={self.k})"
        elif self.type == "logmeanexp":
            s += f"(tau={self.temperature:g})"
        elif self.type == "softmax_weighted":
            s += f"(beta={self.beta:g})"
        elif self.type == "power_mean":
            s += f"(p={self.p:g})"
        if self.activation != "identity":
            s = f"{s}[{self.activation}]"
        if self.out_activation != "identity":
            s = f"{self.out_activation}({s})"
        return s


@dataclass
class PoolingConfig:
    """Pooling levels + checkpoint policy (sparse_pooling/config.py:164-227)."""

    levels: List[LevelSpec]
    checkpoint_policy: str = "auto"
    level1_checkpoint: str = "save"

    def __post_init__(self):
        if not 1 <= len(self.levels) <= 2:
            raise ValueError("1 or 2 pooling levels are supported")
        if self.levels[0].type in LEVEL2_ONLY_TYPES:
            raise ValueError(f"{self.levels[0].type} cannot be a level-1 operator")
        if len(self.levels) == 2:
            if self.levels[0].neurons_per_shard is None:
                raise ValueError("a two-level config needs level-1 neurons_per_shard")
        elif self.levels[0].neurons_per_shard is not None:
            raise ValueError("neurons_per_shard on a single level would change the model; "
                             "use PhysicalPlan for execution-only sharding")
        if self.checkpoint_policy not in CHECKPOINT_POLICIES:
            raise ValueError(f"unknown checkpoint policy {self.checkpoint_policy!r}")
        if self.level1_checkpoint not in ("save", "recompute"):
            raise ValueError("level1_checkpoint must be 'save' or 'recompute'")

    @property
    def is_semantic_hierarchy(self) -> bool:
        return len(self.levels) == 2

    @staticmethod
    def parse(spec: Union[str, Dict[str, Any], "PoolingConfig"], checkpoint_policy: str = "auto"):
        if isinstance(spec, PoolingConfig):
            return spec
        if isinstance(spec, str):
            return PoolingConfig([LevelSpec(type=spec)], checkpoint_policy=checkpoint_policy)
        if isinstance(spec, dict):
            if "levels" in spec:
                levels = [LevelSpec(**lv) for lv in spec["levels"]]
                return PoolingConfig(levels, checkpoint_policy=spec.get("checkpoint_policy", checkpoint_policy),
                                     level1_checkpoint=spec.get("level1_checkpoint", "save"))
            return PoolingConfig([LevelSpec(**spec)], checkpoint_policy=checkpoint_policy)
        raise TypeError(f"cannot parse pooling spec {spec!r}")

    def describe(self) -> str:
        return " -> ".join(lv.describe() for lv in self.levels)


REDUCTIONS = ("auto", "fast", "deterministic")
# the reference's default workspace_budget (sparse_pooling/config.py); a layer built here without a
# budget (None) uses the library's larger defaults instead, an explicit value is always honoured
DEFAULT_WORKSPACE_BUDGET = 512 * 2**20


def check_workspace_budget(budget):
    """None (no budget: the library's defaults) or a positive number of bytes."""
    if budget is None:
        return None
    if isinstance(budget, bool) or int(budget) != budget or int(budget) <= 0:
        raise ValueError(f"workspace_budget must be None or a positive number of bytes (got {budget!r})")
    return int(budget)


@dataclass
class PhysicalPlan:
    """Execution-only plan (sparse_pooling/config.py:240-390).

    The generic fields keep the reference's meaning.  ``backend`` additionally accepts
    ``"hip"``; the reference's ``"cuda"`` / ``"auto"`` select the HIP backend on a ROCm device
    and ``"triton"`` is refused (there is no Triton path).  The CUDA-kernel tuning fields are
    accepted for source compatibility and ignored: the HIP kernels pick their own tiles.  Every
    HIP reduction has a fixed owner and order, so ``reduction="fast"`` and ``"deterministic"``
    both run deterministic kernels.

    ``relu_bits`` is this build's own: ``"recompute"`` (default, the reference's behaviour) keeps
    only the pooled statistics between forward and backward and the backward recomputes z;
    ``"keep"`` also keeps the forward's ReLU bit of every (token, neuron) -- 1/32 of the [B, N]
    hidden tensor's fp32 bytes -- for ReLU mean / sum layers at fan-in 8, so the backward's dW
    pass skips the recompute (same results, bit for bit).
    """

    phys_splits: int = 0
    block_m: int = 64
    num_warps: int = 4
    num_stages: int = 2
    token_tiles_per_program: int = 1
    input_layout: str = "feature_major"
    backend: str = "auto"
    tuning_profile: str = "auto"
    cuda_block_m: int = 32
    cuda_warps: int = 16
    grad_precision: str = "split"
    cuda_dx_epilogue: str = "auto"
    cuda_dw_epilogue: str = "auto"
    cuda_dx_warps: int = 0
    cuda_dw_cfg: int = -1
    cuda_dw_staging: str = "auto"
    cuda_input_supergroup_backend: str = "auto"
    cuda_grouped_fwd: str = ""
    cuda_grouped_dx: str = ""
    cuda_grouped_dw: str = ""
    cuda_grouped_fwd_tokens: int = 0
    cuda_grouped_fwd_warps: int = 0
    cuda_grouped_fwd_chunk_units: int = 0
    cuda_grouped_dx_tokens: int = 0
    cuda_grouped_dx_warps: int = 0
    cuda_grouped_dx_reduction: int = 0
    cuda_grouped_dx_chunk_units: int = 0
    cuda_grouped_dx_scatter: str = "auto"
    cuda_grouped_dx_plan: str = "auto"
    cuda_grouped_backward: str = "auto"
    cuda_grouped_fused_cfg: int = 0
    cuda_grouped_dw_cfg: int = -1
    cuda_grouped_dw_projection: str = "auto"
    cuda_grouped_merge: str = "atomic"
    reduction: str = "auto"
    deterministic_workspace_bytes: int = 0
    relu_bits: str = "recompute"

    def __post_init__(self):
        if self.input_layout not in ("feature_major", "token_major"):
            raise ValueError("input_layout must be 'feature_major' or 'token_major'")
        if self.backend not in ("triton", "cuda", "auto", "hip"):
            raise ValueError("backend must be 'hip', 'cuda', 'auto' or 'triton'")
        if not isinstance(self.tuning_profile, str) or not self.tuning_profile:
            raise ValueError("tuning_profile must be 'auto' or a registered profile name")
        if self.reduction not in REDUCTIONS:
            raise ValueError(f"reduction must be one of {REDUCTIONS} (got {self.reduction!r})")
        if self.deterministic_workspace_bytes < 0:
            raise ValueError("deterministic_workspace_bytes must be >= 0")
        if self.relu_bits not in ("recompute", "keep"):
            raise ValueError(f"relu_bits must be 'recompute' or 'keep' (got {self.relu_bits!r})")


def resolve_reduction(plan: PhysicalPlan):
    """(mode, reason, strict) as sparse_pooling/config.py:397-421.  The HIP kernels are
    deterministic by construction, so no combination is refused for lack of determinism."""
    import torch

    glob = torch.are_deterministic_algorithms_enabled()
    if plan.reduction == "deterministic":
        return "deterministic", "explicit reduction='deterministic'", True
    if plan.reduction == "fast":
        return "fast", "explicit reduction='fast' (HIP reductions are deterministic anyway)", False
    if glob:
        return "deterministic", "torch.use_deterministic_algorithms(True)", True
    return "fast", "default (HIP reductions are deterministic anyway)", False
