"""Neuron layout: partition of H logical neurons into G pools ("groups") of padded slots.

Mirrors the public semantics of sparse_pooling/layout.py (Mode A, independent index records):

    indices [G, NB, C, K] int32     weights [G, NB, C, K]     bias [G, NB, C]

Group g owns n_g = H // G + (g < H % G) valid neurons; slot s = blk * C + c of group g is valid
iff s < n_g and is then the global neuron offset_g + s with offset_g = g * (H // G) + min(g, H % G)
(layout.py:68-120).  NB = ceil(max_group / C) padded to a multiple of 4 blocks, so a group has
S = NB * C slots, a multiple of 32.  Padded slots carry zero weights, bias and indices.

Differences from the reference (recorded in DESIGN.md):
  * indices are stored as int32 (the reference uses int16 and caps input_dim at 32767);
    ``load_int16_indices`` widens a reference checkpoint losslessly;
  * fan_in may be 8 or 16 (16 = the per-neuron K16 compact variant);
  * the mma-fragment "packed" storage exists only for Mode B in the reference and is not
    provided here (Mode B is not on the MI355X path).
"""
from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class SparseLayout:
    input_dim: int
    hidden_dim: int
    groups: int
    fan_in: int
    block: int
    shared_indices: bool
    packed: bool = False

    def __post_init__(self):
        if self.fan_in not in (8, 16):
            raise ValueError("fan-in must be 8 (or 16 for the per-neuron K16 variant)")
        if self.input_dim < 1 or self.input_dim > 2**31 - 1:
            raise ValueError("input_dim must be in [1, 2^31 - 1] (int32 indices)")
        if self.block not in (8, 16, 32, 64):
            raise ValueError("block (shared_neurons) must be 8, 16, 32 or 64")
        if self.hidden_dim < self.groups:
            raise ValueError("need at least one neuron per group")
        if self.packed and not self.shared_indices:
            raise ValueError("fragment-packed storage is only defined for Mode B")
        if self.packed:
            raise NotImplementedError("fragment-packed (Mode B, mma) storage is not on the MI355X path")

    # ---- partition -------------------------------------------------------
    @property
    def base(self) -> int:
        return self.hidden_dim // self.groups

    @property
    def rem(self) -> int:
        return self.hidden_dim % self.groups

    @property
    def max_group(self) -> int:
        return self.base + (1 if self.rem else 0)

    @property
    def blocks_per_group(self) -> int:
        nb = -(-self.max_group // self.block)
        return (nb + 3) // 4 * 4

    @property
    def slots_per_group(self) -> int:
        return self.blocks_per_group * self.block

    def group_count(self, g: int) -> int:
        return self.base + (1 if g < self.rem else 0)

    def group_offset(self, g: int) -> int:
        return g * self.base + min(g, self.rem)

    def counts_tensor(self, device) -> torch.Tensor:
        g = torch.arange(self.groups, device=device)
        return (self.base + (g < self.rem).to(torch.int64)).to(torch.int32)

    def offsets_tensor(self, device) -> torch.Tensor:
        g = torch.arange(self.groups, device=device, dtype=torch.int64)
        return g * self.base + torch.clamp(g, max=self.rem)

    def global_ids(self, device) -> torch.Tensor:
        """[G, slots] int64 global neuron id, -1 for padded slots."""
        s = torch.arange(self.slots_per_group, device=device, dtype=torch.int64)
        ids = self.offsets_tensor(device)[:, None] + s[None, :]
        valid = s[None, :] < self.counts_tensor(device)[:, None].to(torch.int64)
        return torch.where(valid, ids, torch.full_like(ids, -1))

    def valid_mask(self, device) -> torch.Tensor:
        s = torch.arange(self.slots_per_group, device=device)
        return s[None, :] < self.counts_tensor(device)[:, None]

    # ---- shapes ----------------------------------------------------------
    @property
    def index_shape(self):
        G, NB, C, K = self.groups, self.blocks_per_group, self.block, self.fan_in
        return (G, NB, K) if self.shared_indices else (G, NB, C, K)

    @property
    def weight_shape(self):
        return (self.groups, self.blocks_per_group, self.block, self.fan_in)

    @property
    def bias_shape(self):
        return (self.groups, self.blocks_per_group, self.block)

    @property
    def canonical(self) -> "SparseLayout":
        return dataclasses.replace(self, packed=False)

    def to_canonical(self, idx, w, b):
        return idx, w, b

    def param_bytes(self, dtype_bytes: int = 4) -> dict:
        return {"weights": math.prod(self.weight_shape) * dtype_bytes, "bias": math.prod(self.bias_shape) * dtype_bytes,
                "indices": math.prod(self.index_shape) * 4}

    def padding_fraction(self) -> float:
        return 1.0 - self.hidden_dim / (self.groups * self.slots_per_group)


def sample_distinct(n_rec: int, d: int, k: int, gen: torch.Generator, device, low: int = 0) -> torch.Tensor:
    """n_rec records of k distinct indices in [low, low + d), sorted ascending (int64).

    Same procedure as the reference's _sample_distinct (layout.py:191-201): draw uniformly,
    sort every record, redraw the records that contain a repeat until none does."""
    if k > d:
        raise ValueError(f"cannot draw {k} distinct indices from {d} values")
    out = torch.randint(0, d, (n_rec, k), generator=gen, device=device, dtype=torch.int64)
    while True:
        out, _ = torch.sort(out, dim=1)
        dup = (out[:, 1:] == out[:, :-1]).any(dim=1)
        nd = int(dup.sum())
        if nd == 0:
            break
        out[dup] = torch.randint(0, d, (nd, k), generator=gen, device=device, dtype=torch.int64)
    return out + low


@torch.no_grad()
def init_parameters(layout: SparseLayout, device, dtype=torch.float32, seed: int = 0, weight_std: float | None = None,
                    bias_std: float = 0.0, chunk_records: int = 1 << 22):
    """(indices int32, weights, bias) with padded slots zeroed (layout.py:204-251 semantics:
    distinct sorted records, weights N(0, weight_std^2) with default std 1/sqrt(K), bias zero or
    N(0, bias_std^2)); generated in chunks so 100M-neuron layers need no large temporaries."""
    if layout.shared_indices:
        raise NotImplementedError("Mode B (block-shared indices) is not on the MI355X path")
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    K = layout.fan_in
    if weight_std is None:
        weight_std = 1.0 / math.sqrt(K)
    idx = torch.empty(layout.index_shape, dtype=torch.int32, device=device)
    flat_idx = idx.view(-1, K)
    for s in range(0, flat_idx.shape[0], chunk_records):
        e = min(s + chunk_records, flat_idx.shape[0])
        flat_idx[s:e] = sample_distinct(e - s, layout.input_dim, K, gen, device).to(torch.int32)
    w = torch.empty(layout.weight_shape, dtype=dtype, device=device)
    flat_w = w.view(-1)
    step = chunk_records * K
    for s in range(0, flat_w.numel(), step):
        e = min(s + step, flat_w.numel())
        flat_w[s:e] = (torch.randn(e - s, generator=gen, device=device) * weight_std).to(dtype)
    b = torch.empty(layout.bias_shape, dtype=dtype, device=device)
    if bias_std > 0:
        b.copy_((torch.randn(b.shape, generator=gen, device=device) * bias_std).to(dtype))
    else:
        b.zero_()
    zero_padding_(layout, weights=w, bias=b, indices=idx)
    return idx, w, b


@torch.no_grad()
def zero_padding_(layout: SparseLayout, weights=None, bias=None, indices=None):
    """Zero the padded slots of weights [G,NB,C,K], bias [G,NB,C] and Mode-A indices."""
    ref = next(t for t in (weights, bias, indices) if t is not None)
    G, NB, C = layout.groups, layout.blocks_per_group, layout.block
    counts = layout.counts_tensor(ref.device).to(torch.int64)
    slots = torch.arange(NB * C, device=ref.device)
    invalid = (slots[None, :] >= counts[:, None]).view(G, NB, C)
    if weights is not None:
        weights.masked_fill_(invalid[..., None], 0)
    if bias is not None:
        bias.masked_fill_(invalid, 0)
    if indices is not None and not layout.shared_indices:
        indices.masked_fill_(invalid[..., None], 0)


def check_indices(layout: SparseLayout, idx: torch.Tensor) -> None:
    """Refuse indices outside [0, input_dim) in valid slots (the kernels would otherwise clamp)."""
    if idx.dtype != torch.int32:
        raise TypeError(f"indices must be int32 (got {idx.dtype}); widen int16 reference checkpoints with "
                        "load_int16_indices")
    if tuple(idx.shape) != tuple(layout.index_shape):
        raise ValueError(f"indices shape {tuple(idx.shape)} != layout {layout.index_shape}")
    flat = idx.view(layout.groups, -1, layout.fan_in)
    valid = layout.valid_mask(idx.device)
    lo = int(torch.where(valid[..., None], flat, torch.zeros_like(flat)).min())
    hi = int(torch.where(valid[..., None], flat, torch.zeros_like(flat)).max())
    if lo < 0 or hi >= layout.input_dim:
        raise ValueError(f"indices must lie in [0, {layout.input_dim}) (found [{lo}, {hi}])")


def load_int16_indices(idx16: torch.Tensor) -> torch.Tensor:
    """Widen a reference (int16) index tensor to this layout's int32 storage, value for value."""
    if idx16.dtype != torch.int16:
        raise TypeError("expected an int16 index tensor")
    return idx16.to(torch.int32)
