"""Cover-TopK/16: a frozen 16-input support per 16-neuron row group, selected once from a K64
envelope and executed compactly with one K16 index record per 16 neurons.  Mirrors
sparse_pooling/cover_topk16.py (CoverTopK16Layer, :1-264) and the selection of
sparse_pooling/experimental/local_supports.py (feature_importance :209-222, topk_select :279-282,
cover_repair :294-375).

Envelope (input of ``from_envelope``): output g owns n_g = H // G + (g < H % G) neurons in NB
records of C neurons (C a multiple of 16, 256 by default; ``EnvelopeLayout``, the partition of
sparse_pooling/experimental/kgen_layout.py:28-101); every record (g, j) shares 64 candidate inputs
``env_indices[g, j]`` and each of its neurons has 64 weights.  Selection, per 16-neuron row group
u = (g, j, c // 16), runs in the HIP kernel ``gl_cover_select``:

1. importance a[u, i] = sum over u's valid neurons of W[u, c, i]^2 (float64, neuron order);
2. TopK: the 16 largest a[u, i], ties to the lower candidate position;
3. cover repair: every candidate of a record is kept by at least one of its valid groups, by
   greedy minimum-energy-loss swaps (records with m valid groups and 16 m < 64 are refused);
4. every valid neuron keeps its 16 weights at its group's kept positions and its own bias; the
   per-output valid-neuron count (the Mean denominator) is unchanged;
5. optional one-time energy restoration (``normalization="energy"``,
   experimental/row_normalize.py): s_i = min(8, sqrt(E_dense_i / max(E_kept_i, 1e-6 E_dense_i))) per
   neuron over its 64 envelope weights, weights only, applied once before execution.

Execution: the layer is a Mode-A-shaped layer of S = NB C slots per output whose index records
are shared by 16 consecutive slots (``rec_shift`` 4 in the C ABI): the forward and dW kernels load
one record per row group (the 16 lanes of a row group read the same LDS addresses), dX walks the
per-neuron edges.  fp32 parameters, Mean(ReLU) by default (any pooling the HIP path runs),
recompute backward, fp32 ``main_grad``.
"""
from __future__ import annotations

import ctypes
import hashlib
import math
import time
from dataclasses import dataclass
from pathlib import Path
from typing import Optional, Union

import torch
from torch import nn

from . import _native as N
from .autograd import Level1Runtime, SparsePoolFunction, resolve_policy
from .config import PhysicalPlan, PoolingConfig, check_workspace_budget

POLICY = "Cover-TopK"
FAN_IN = 16
CANDIDATES = 64
SCHEMA = "granulelayer_amd.cover_topk16/1"
PACKED_SCHEMA = "granulelayer_amd.cover_topk16_packed/1"
NORMALIZATIONS = ("none", "energy")
S_MAX, EPS_REL = 8.0, 1e-6  # energy restoration clip and relative floor (row_normalize.py)


@dataclass(frozen=True)
class EnvelopeLayout:
    """Partition of a K64 envelope: output g owns n_g = H // G + (g < H % G) neurons, in NB =
    ceil(max n_g / C) records of C neurons; slot s = j C + c of output g is valid iff s < n_g."""

    input_dim: int
    hidden_dim: int
    groups: int
    fan_in: int = CANDIDATES
    block: int = 256

    def __post_init__(self):
        if self.fan_in != CANDIDATES:
            raise ValueError(f"Cover-TopK/16 selects from {CANDIDATES} candidates (fan_in {self.fan_in})")
        if self.block % 16 or not 16 <= self.block <= 256:
            raise ValueError(f"envelope C must be a multiple of 16 in [16, 256] (got {self.block})")
        if self.hidden_dim < self.groups:
            raise ValueError("need at least one neuron per group")

    @property
    def max_group(self) -> int:
        return self.hidden_dim // self.groups + (1 if self.hidden_dim % self.groups else 0)

    @property
    def blocks_per_group(self) -> int:
        return math.ceil(self.max_group / self.block)

    @property
    def slots_per_group(self) -> int:
        return self.blocks_per_group * self.block

    def counts_tensor(self, device) -> torch.Tensor:
        g = torch.arange(self.groups, device=device)
        return (self.hidden_dim // self.groups + (g < self.hidden_dim % self.groups).to(torch.int64)).to(torch.int32)

    def valid_mask(self, device) -> torch.Tensor:
        s = torch.arange(self.slots_per_group, device=device)
        return (s[None, :] < self.counts_tensor(device)[:, None]).view(self.groups, self.blocks_per_group, self.block)

    def record_counts(self, device) -> torch.Tensor:
        """[G NB] valid neurons of every record (0..C)."""
        j = torch.arange(self.blocks_per_group, device=device, dtype=torch.int64)
        n = self.counts_tensor(device).to(torch.int64)[:, None] - j[None, :] * self.block
        return n.clamp(0, self.block).reshape(-1).to(torch.int32)

    @property
    def index_shape(self):
        return (self.groups, self.blocks_per_group, CANDIDATES)

    @property
    def weight_shape(self):
        return (self.groups, self.blocks_per_group, self.block, CANDIDATES)

    @property
    def bias_shape(self):
        return (self.groups, self.blocks_per_group, self.block)


@dataclass(frozen=True)
class CompactLayout:
    """Execution layout of the compact layer: S slots per output, one K16 index record per 16
    consecutive slots.  Shapes: indices [G, S/16, 16], weight [G, S/16, 16, 16] (row group, neuron,
    kept input), bias [G, S/16, 16]; the kernels see W as [G S, 16] and records as [G S / 16, 16]."""

    input_dim: int
    hidden_dim: int
    groups: int
    slots_per_group: int
    fan_in: int = FAN_IN
    rec_shift: int = 4
    shared_indices: bool = True

    @property
    def rows_per_group(self) -> int:
        return self.slots_per_group // 16

    @property
    def blocks_per_group(self) -> int:
        return self.rows_per_group

    def counts_tensor(self, device) -> torch.Tensor:
        g = torch.arange(self.groups, device=device)
        return (self.hidden_dim // self.groups + (g < self.hidden_dim % self.groups).to(torch.int64)).to(torch.int32)

    def valid_mask(self, device) -> torch.Tensor:
        s = torch.arange(self.slots_per_group, device=device)
        return (s[None, :] < self.counts_tensor(device)[:, None]).view(self.groups, self.rows_per_group, 16)

    @property
    def index_shape(self):
        return (self.groups, self.rows_per_group, FAN_IN)

    @property
    def weight_shape(self):
        return (self.groups, self.rows_per_group, 16, FAN_IN)

    @property
    def bias_shape(self):
        return (self.groups, self.rows_per_group, 16)


# ---------------------------------------------------------------------------- selection API
def _ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.data_ptr()


def _select(W=None, a=None, nvalid=None, cand=None, R=0, gpb=1, k=FAN_IN, repair=True, want_importance=False,
            want_weights=False, device=None):
    """Run gl_cover_select; returns the outputs asked for (device tensors)."""
    dev = device or (W.device if W is not None else a.device)
    if dev.type != "cuda":
        raise RuntimeError("Cover-TopK selection runs on a ROCm GPU (the HIP kernel gl_cover_select)")
    out = {"env": torch.empty((R * gpb, k), dtype=torch.int32, device=dev),
           "missing0": torch.empty(R, dtype=torch.int32, device=dev),
           "swaps": torch.empty(R, dtype=torch.int32, device=dev),
           "loss": torch.empty(R, dtype=torch.float64, device=dev),
           "status": torch.empty(R, dtype=torch.int32, device=dev)}
    if want_importance:
        out["importance"] = torch.empty((R * gpb, CANDIDATES), dtype=torch.float64, device=dev)
    if cand is not None:
        out["rec_idx"] = torch.empty((R * gpb, k), dtype=torch.int32, device=dev)
    if want_weights:
        out["W_out"] = torch.empty((R * gpb * 16, k), dtype=torch.float32, device=dev)
    args = N.GlCoverArgs(W=_ptr(W), a=_ptr(a), nvalid=_ptr(nvalid), cand=_ptr(cand), R=R, gpb=gpb, k=k,
                         repair=int(repair), importance=_ptr(out.get("importance")), env=_ptr(out["env"]),
                         rec_idx=_ptr(out.get("rec_idx")), W_out=_ptr(out.get("W_out")),
                         missing0=_ptr(out["missing0"]), swaps=_ptr(out["swaps"]), loss=_ptr(out["loss"]),
                         status=_ptr(out["status"]))
    lib = N.library()
    with torch.cuda.device(dev):
        lib.call("gl_cover_select", ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    return out


def _records(w: torch.Tensor, L: EnvelopeLayout):
    if tuple(w.shape) != tuple(L.weight_shape):
        raise ValueError(f"envelope weights must be {L.weight_shape} (got {tuple(w.shape)})")
    W = w.detach().to(torch.float32).contiguous()
    return W, L.record_counts(W.device), L.groups * L.blocks_per_group, L.block // 16


@torch.no_grad()
def feature_importance(w: torch.Tensor, L: EnvelopeLayout) -> torch.Tensor:
    """[n16, 64] float64 a[u, i] = sum over the valid neurons c of row group u of W[u, c, i]^2, added
    in order c = 0..15 (local_supports.py:209-222); n16 = G NB C / 16."""
    W, nvalid, R, gpb = _records(w, L)
    return _select(W=W, nvalid=nvalid, R=R, gpb=gpb, repair=False, want_importance=True)["importance"]


@torch.no_grad()
def topk_select(a_v: torch.Tensor, k: int) -> torch.Tensor:
    """[n, k] int64 sorted positions of the k largest of each row of a_v [n, 64] (float64), ties to
    the lower position (local_supports.py:279-282)."""
    a = a_v.to(torch.float64).contiguous()
    if a.dim() != 2 or a.shape[1] != CANDIDATES:
        raise ValueError("a_v must be [n, 64]")
    n = a.shape[0]
    nvalid = torch.full((n,), 16, dtype=torch.int32, device=a.device)
    return _select(a=a, nvalid=nvalid, R=n, gpb=1, k=k, repair=False)["env"].to(torch.int64)


@torch.no_grad()
def cover_topk(w: torch.Tensor, L: EnvelopeLayout, env_indices: Optional[torch.Tensor] = None, k: int = FAN_IN,
               repair: bool = True) -> dict:
    """Cover-TopK supports of an envelope: env [n16, k] kept positions of every row group (padded
    groups: 0..k-1), rec_idx (the kept global inputs, when env_indices [G, NB, 64] is given), W_out
    [n16 16, k] every neuron's kept weights, and per record missing0 / swaps / loss (float64).
    Records with m valid groups and m k < 64 raise ValueError, as the reference's cover_repair."""
    W, nvalid, R, gpb = _records(w, L)
    cand = None
    if env_indices is not None:
        if tuple(env_indices.shape) != tuple(L.index_shape):
            raise ValueError(f"env_indices must be {L.index_shape}")
        cand = env_indices.to(device=W.device, dtype=torch.int32).contiguous()
    out = _select(W=W, nvalid=nvalid, cand=cand, R=R, gpb=gpb, k=k, repair=repair, want_weights=True)
    bad = torch.nonzero(out["status"] != 0)
    if bad.numel():
        r = int(bad[0, 0])
        m = (int(nvalid[r]) + 15) // 16
        raise ValueError(f"Cover-TopK infeasible: record {r} has {m} valid groups and k = {k} (m k = {m * k} < "
                         f"{CANDIDATES}); no epsilon edges / padding / larger k are used")
    return out


def _energy_scales(W: torch.Tensor, W_kept: torch.Tensor, valid: torch.Tensor) -> torch.Tensor:
    """Per neuron s = min(8, sqrt(E_dense / max(E_kept, 1e-6 E_dense))) from fp32 sums of its 64
    envelope weights and of its kept ones; 1 for an all-zero row, 0 for padded neurons
    (experimental/row_normalize.py:row_scales, treatment "energy")."""
    e = (W * W).sum(1)
    ek = (W_kept * W_kept).sum(1)
    s = torch.clamp(torch.sqrt(e / torch.maximum(ek, EPS_REL * e)), max=S_MAX)
    s = torch.where(e > 0, s, torch.ones_like(s))
    return torch.where(valid, s, torch.zeros_like(s))


def tensor_sha256(t: torch.Tensor) -> str:
    h = hashlib.sha256()
    h.update(t.detach().contiguous().cpu().numpy().tobytes())
    return h.hexdigest()


# ---------------------------------------------------------------------------- layer
class CoverTopK16Layer(nn.Module):
    """The Cover-TopK/16 layer (module docstring).  Build with ``from_envelope``, restore with
    ``load_packed``; ``forward`` accepts [..., D] and returns [..., G]."""

    def __init__(self, input_dim: int, hidden_dim: int, output_dim: int, slots_per_group: int, *,
                 pooling: Union[str, dict, PoolingConfig] = "mean", checkpoint_policy: str = "auto",
                 plan: Optional[PhysicalPlan] = None, workspace_budget: Optional[int] = None, device=None):
        super().__init__()
        if slots_per_group % 16:
            raise ValueError("slots_per_group must be a multiple of 16")
        self.layout = CompactLayout(input_dim, hidden_dim, output_dim, slots_per_group)
        if int(self.layout.counts_tensor("cpu").max()) > slots_per_group:
            raise ValueError("slots_per_group is smaller than the largest output's neuron count")
        self.cfg = PoolingConfig.parse(pooling, checkpoint_policy)
        if isinstance(pooling, (str, PoolingConfig)) or "checkpoint_policy" not in (pooling or {}):
            self.cfg.checkpoint_policy = checkpoint_policy
        if self.cfg.is_semantic_hierarchy:
            raise NotImplementedError("semantic two-level pooling is not on the MI355X path")
        reason = self.cfg.levels[0].hip_reason()
        if reason:
            raise NotImplementedError(reason)
        self.plan = plan or PhysicalPlan()
        self.workspace_budget = check_workspace_budget(workspace_budget)
        self.compute_dtype = torch.float32
        L = self.layout
        dev = device or "cpu"
        self.register_buffer("indices", torch.zeros(L.index_shape, dtype=torch.int32, device=dev))
        self.register_buffer("env", torch.zeros(L.index_shape, dtype=torch.int32, device=dev))
        self.weight = nn.Parameter(torch.zeros(L.weight_shape, dtype=torch.float32, device=dev))
        self.bias = nn.Parameter(torch.zeros(L.bias_shape, dtype=torch.float32, device=dev))
        self.cover_meta: dict = {}
        self._rt = None
        self._rt_key = None

    # ------------------------------------------------------------------ construction
    @classmethod
    @torch.no_grad()
    def from_envelope(cls, weight: torch.Tensor, bias: torch.Tensor, env_indices: torch.Tensor, *, input_dim: int,
                      hidden_dim: int, output_dim: int, envelope_C: int = 256, normalization: str = "none",
                      pooling="mean", plan: Optional[PhysicalPlan] = None, device=None) -> "CoverTopK16Layer":
        """Select the Cover-TopK/16 support from K64 envelope values and build the compact layer.

        ``weight`` [G, NB, envelope_C, 64] / ``bias`` [G, NB, envelope_C]: the pre-pruning envelope
        values in ``EnvelopeLayout(input_dim, hidden_dim, output_dim, 64, envelope_C)`` order;
        ``env_indices`` [G, NB, 64]: the 64 candidate inputs of every record (distinct, in
        [0, input_dim)).  The caller's tensors are not modified.  (The reference regenerates the
        envelope graph from a ConnectivityPlan, cover_topk16.py:80-118; here the graph is given.)"""
        if normalization not in NORMALIZATIONS:
            raise ValueError(f"normalization {normalization!r} (one of {NORMALIZATIONS})")
        L = EnvelopeLayout(input_dim, hidden_dim, output_dim, CANDIDATES, envelope_C)
        dev = torch.device(device) if device is not None else weight.device
        if tuple(bias.shape) != tuple(L.bias_shape) or tuple(env_indices.shape) != tuple(L.index_shape):
            raise ValueError(f"bias must be {L.bias_shape} and env_indices {L.index_shape}")
        cand = env_indices.to(dev, torch.int32)
        valid_rec = L.record_counts(dev) > 0
        ci = cand.view(-1, CANDIDATES)[valid_rec]
        if ci.numel() and (int(ci.min()) < 0 or int(ci.max()) >= input_dim):
            raise ValueError(f"env_indices must lie in [0, {input_dim})")
        if ci.numel() and bool((torch.sort(ci, 1).values[:, 1:] == torch.sort(ci, 1).values[:, :-1]).any()):
            raise ValueError("the 64 candidates of a record must be distinct")
        t0 = time.perf_counter()
        w = weight.detach().to(dev, torch.float32)
        sel = cover_topk(w, L, cand, FAN_IN, repair=True)
        torch.cuda.synchronize(dev)
        sel_s = time.perf_counter() - t0
        W_kept = sel["W_out"]  # [G NB C, 16]
        valid = L.valid_mask(dev).reshape(-1)
        nrec = dict(treatment="none", applied=False)
        if normalization == "energy":
            kept_mask = torch.zeros((W_kept.shape[0], CANDIDATES), dtype=torch.bool, device=dev)
            grp = sel["env"].to(torch.int64).repeat_interleave(16, 0)  # every neuron's kept positions
            kept_mask.scatter_(1, grp, True)
            Wd = w.reshape(-1, CANDIDATES)
            s = _energy_scales(Wd, Wd * kept_mask, valid)
            W_kept = W_kept * s[:, None]
            nrec = dict(treatment="energy", applied=True, s_max=S_MAX, eps_rel=EPS_REL,
                        clipped=int((s == S_MAX).sum()), scale_mean=float(s[valid].mean()))
        S = L.slots_per_group
        lay = cls(input_dim, hidden_dim, output_dim, S, pooling=pooling, plan=plan, device=dev)
        lay.indices.copy_(sel["rec_idx"].view(lay.layout.index_shape))
        lay.env.copy_(sel["env"].view(lay.layout.index_shape))
        lay.weight.copy_(W_kept.view(lay.layout.weight_shape))
        b = bias.detach().to(dev, torch.float32).reshape(-1) * valid
        lay.bias.copy_(b.view(lay.layout.bias_shape))
        lay.cover_meta = dict(
            schema=SCHEMA, policy=POLICY, fan_in=FAN_IN,
            envelope=dict(K=CANDIDATES, C=envelope_C, records=int(valid_rec.sum())),
            executed=dict(K=FAN_IN, C=16, records_16=int((lay.layout.valid_mask("cpu").reshape(-1, 16).any(1)).sum())),
            input_dim=input_dim, hidden_dim=hidden_dim, output_dim=output_dim,
            valid_slots=FAN_IN * hidden_dim, biases=hidden_dim,
            support_fingerprint=tensor_sha256(sel["env"]),
            support_stats=dict(missing0=int(sel["missing0"].sum()), swaps=int(sel["swaps"].sum()),
                               energy_loss=float(sel["loss"].sum()), max_swaps=int(sel["swaps"].max())),
            normalization=nrec, normalization_scale_bias=False,
            construction_seconds=dict(selection=sel_s))
        return lay

    # ------------------------------------------------------------------ persistence
    def immutable_fingerprints(self) -> dict:
        return {"indices": tensor_sha256(self.indices), "env": tensor_sha256(self.env)}

    def save_packed(self, path) -> dict:
        """Save the frozen compact layer: records, kept positions, weights, bias, layout, pooling,
        metadata and the fingerprints of the immutable buffers (the reference's save_packed,
        cover_topk16.py:196-212).  The optimizer state is saved separately."""
        L = self.layout
        blob = dict(schema=PACKED_SCHEMA, meta=self.cover_meta,
                    layout=dict(input_dim=L.input_dim, hidden_dim=L.hidden_dim, output_dim=L.groups,
                                slots_per_group=L.slots_per_group, fan_in=L.fan_in, C=16),
                    pooling=self.cfg.levels[0].describe(), fingerprints=self.immutable_fingerprints(),
                    state={k: v.detach().cpu() for k, v in self.state_dict().items()})
        Path(path).parent.mkdir(parents=True, exist_ok=True)
        torch.save(blob, path)
        return dict(path=str(path), fingerprints=blob["fingerprints"])

    @classmethod
    def load_packed(cls, path, *, device=None, pooling="mean", plan: Optional[PhysicalPlan] = None
                    ) -> "CoverTopK16Layer":
        """Restore a ``save_packed`` file (no selection, no envelope needed), refusing files whose
        immutable buffers differ from their recorded fingerprints (cover_topk16.py:214-236)."""
        blob = torch.load(Path(path), map_location="cpu", weights_only=True)
        if blob.get("schema") != PACKED_SCHEMA:
            raise ValueError(f"{path}: schema {blob.get('schema')!r}, expected {PACKED_SCHEMA!r}")
        lo = blob["layout"]
        lay = cls(lo["input_dim"], lo["hidden_dim"], lo["output_dim"], lo["slots_per_group"], pooling=pooling,
                  plan=plan, device=device)
        lay.load_state_dict(blob["state"])
        lay.cover_meta = blob["meta"]
        if lay.immutable_fingerprints() != blob["fingerprints"]:
            raise ValueError(f"{path}: immutable buffers differ from their recorded fingerprints")
        return lay

    # ------------------------------------------------------------------ execution
    @property
    def metadata(self) -> dict:
        return self.cover_meta

    @property
    def normalization(self) -> dict:
        return self.cover_meta.get("normalization", {})

    def _load_from_state_dict(self, *args, **kwargs):
        super()._load_from_state_dict(*args, **kwargs)
        self._rt = None

    def _runtime(self) -> Level1Runtime:
        key = (self.indices.device, self.indices.data_ptr(), self.indices._version, id(self.plan))
        if self._rt is None or self._rt_key != key:
            self._rt = Level1Runtime(self.layout, self.indices, self.cfg.levels[0], self.plan, None,
                                     self.workspace_budget, None)
            self._rt_key = key
        return self._rt

    @property
    def last_info(self):
        return {} if self._rt is None else dict(self._rt.last_info)

    @property
    def effective_policy(self) -> str:
        return resolve_policy(self.cfg.levels[0], self.cfg.checkpoint_policy)

    def enable_main_grad(self):
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
        rt.grad_call = torch.is_grad_enabled()
        y = SparsePoolFunction.apply(x2, self.weight, self.bias, rt, self.effective_policy,
                                     self.compute_dtype)
        return y.reshape(*lead, y.shape[-1])

    def extra_repr(self) -> str:
        L = self.layout
        return (f"Cover-TopK/16: in={L.input_dim}, hidden={L.hidden_dim:,}, out={L.groups}, executed K16/C16, "
                f"pooling={self.cfg.describe()}, normalization={self.normalization.get('treatment', 'none')}")
