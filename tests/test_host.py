"""Host logic on the CPU: layout partition, parameter initialisation, configuration parsing,
refusal of configurations outside the MI355X path, and the synthetic BASELINE generators.
Mirrors the reference's host-only tests (tests/test_sparse_projection.py:14-51)."""
import math

import numpy as np
import pytest
import torch

from granulelayer_amd import FusedAdamW, LevelSpec, PhysicalPlan, PoolingConfig, SparseLayout, SparsePoolingLayer
from granulelayer_amd.autograd import Level1Runtime
from granulelayer_amd.layout import check_indices, init_parameters, load_int16_indices, zero_padding_
from granulelayer_amd.synthetic import CONFIGS, make_problem


@pytest.mark.parametrize("H,G", [(100_000_000, 1024), (100_663_296, 98_304), (5000, 16), (1000, 7)])
def test_partition_enumerates_exactly_H(H, G):
    L = SparseLayout(1024, H, G, 8, 8, False)
    counts = L.counts_tensor("cpu").long()
    offs = L.offsets_tensor("cpu")
    assert int(counts.sum()) == H
    assert int(offs[0]) == 0
    assert torch.equal(offs[1:], offs[:-1] + counts[:-1])
    assert int(counts.max() - counts.min()) <= 1
    assert L.slots_per_group >= L.max_group and L.blocks_per_group % 4 == 0
    if H < 10**6:
        ids = L.global_ids("cpu")
        assert torch.equal(torch.sort(ids[ids >= 0]).values, torch.arange(H))


def test_baseline_layout_shapes():
    L = SparseLayout(4096, 100_663_296, 98_304, 8, 8, False)
    assert L.index_shape == (98_304, 128, 8, 8)
    assert L.slots_per_group == 1024 and L.padding_fraction() == 0.0
    L5 = SparseLayout(4096, 50_331_648, 98_304, 16, 8, False)
    assert L5.weight_shape == (98_304, 64, 8, 16)


@pytest.mark.parametrize("K", [8, 16])
def test_indices_distinct_sorted_and_padding_zero(K):
    L = SparseLayout(64, 3001, 8, K, 8, False)
    idx, w, b = init_parameters(L, "cpu", seed=1, bias_std=0.5)
    assert idx.dtype == torch.int32
    valid = L.valid_mask("cpu").reshape(-1)
    flat = idx.reshape(-1, K).long()
    v = flat[valid]
    assert int(v.min()) >= 0 and int(v.max()) < 64
    assert bool((v[:, 1:] > v[:, :-1]).all()), "indices must be distinct and sorted"
    assert not flat[~valid].any()
    assert not w.reshape(-1, K)[~valid].any() and not b.reshape(-1)[~valid].any()
    # weight scale 1/sqrt(K)
    assert abs(float(w.reshape(-1, K)[valid].std()) - 1 / math.sqrt(K)) < 0.02
    check_indices(L, idx)


def test_init_is_seeded_and_zero_padding_idempotent():
    L = SparseLayout(128, 5000, 16, 8, 8, False)
    a = init_parameters(L, "cpu", seed=3)
    b = init_parameters(L, "cpu", seed=3)
    c = init_parameters(L, "cpu", seed=4)
    assert all(torch.equal(p, q) for p, q in zip(a, b))
    assert not torch.equal(a[0], c[0])
    idx, w, bias = (t.clone() for t in a)
    zero_padding_(L, weights=w, bias=bias, indices=idx)
    assert torch.equal(w, a[1]) and torch.equal(idx, a[0])


def test_check_indices_refuses_out_of_range_and_int16():
    L = SparseLayout(64, 3000, 8, 8, 8, False)
    idx, _, _ = init_parameters(L, "cpu", seed=0)
    bad = idx.clone()
    bad.view(-1)[0] = 64
    with pytest.raises(ValueError, match=r"\[0, 64\)"):
        check_indices(L, bad)
    with pytest.raises(TypeError, match="int32"):
        check_indices(L, idx.to(torch.int16))
    assert torch.equal(load_int16_indices(idx.to(torch.int16)), idx)


def test_config_parsing_matches_reference_semantics():
    assert PoolingConfig.parse("mean").levels[0].activation == "relu"
    assert PoolingConfig.parse("sum").levels[0].activation == "relu"
    assert PoolingConfig.parse({"type": "mean", "activation": "identity"}).levels[0].hip_reason() == ""
    assert LevelSpec("max").out_activation == "relu"
    assert LevelSpec("max").hip_reason() == ""  # max pooling with winner ids is on the HIP path
    for t in ("logmeanexp", "power_mean", "softmax_weighted"):  # smooth operators are on the HIP path
        assert LevelSpec(t).hip_reason() == ""
    assert LevelSpec("mean", neurons_per_shard=64).hip_reason() == ""  # level-1 shards of two-level pooling
    assert LevelSpec("mean", neurons_per_shard=48).hip_reason()  # not a multiple of 4*C = 32
    assert LevelSpec("mean", out_activation="gelu").hip_reason() == ""  # applied to pre in torch
    for t in ("mean", "sum", "max", "topk_mean", "logmeanexp", "softmax_weighted"):  # GELU neurons run in the kernels
        assert LevelSpec(t, activation="gelu").hip_reason() == ""
    with pytest.raises(ValueError):
        LevelSpec("power_mean", activation="gelu")  # the reference defines the power mean on relu only
    with pytest.raises(ValueError):
        LevelSpec("topk_mean", k=3)
    with pytest.raises(ValueError):
        PhysicalPlan(reduction="sometimes")
    PhysicalPlan(cuda_block_m=16, cuda_warps=8)  # CUDA tuning fields accepted, ignored


@pytest.mark.parametrize("kwargs,exc", [
    (dict(shared_neurons=8, pooling="mean"), NotImplementedError),
    (dict(shared_neurons=None, pooling="mean", connectivity=object()), NotImplementedError),
    (dict(shared_neurons=None, pooling="mean", backend="triton"), ValueError),
    (dict(shared_neurons=None, pooling="mean", weight_layout="packed"), ValueError),
])
def test_layer_refuses_configurations_off_the_path(kwargs, exc):
    with pytest.raises(exc):
        SparsePoolingLayer(64, 3000, 8, dtype=torch.float32, **kwargs)


def test_cpu_layer_has_no_fallback():
    lay = SparsePoolingLayer(64, 3000, 8, shared_neurons=None, pooling="mean", dtype=torch.float32)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        lay(torch.randn(2, 64))
    assert lay.explain()["backend"] == "none (CPU parameters)"


def test_runtime_refuses_triton_plan():
    L = SparseLayout(64, 3000, 8, 8, 8, False)
    idx, _, _ = init_parameters(L, "cpu")
    with pytest.raises(NotImplementedError, match="Triton"):
        Level1Runtime(L, idx, LevelSpec("mean"), PhysicalPlan(backend="triton"))


def test_fused_adamw_refuses_what_it_cannot_update():
    p = torch.nn.Parameter(torch.zeros(8, dtype=torch.float16))  # fp32 and bf16 only
    p.grad = torch.zeros(8, dtype=torch.float16)
    with pytest.raises(NotImplementedError):
        FusedAdamW([p]).step()
    q = torch.nn.Parameter(torch.zeros(8, dtype=torch.bfloat16))  # bf16 is supported, on a ROCm GPU only
    q.grad = torch.zeros(8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        FusedAdamW([q]).step()


@pytest.mark.parametrize("name", list(CONFIGS))
def test_synthetic_problems(name):
    pr = make_problem(name, device="cpu", seed=0, groups=4)
    c = CONFIGS[name]
    L = pr.layout
    K, D, pool = c["K"], c["D"], c["pool"]
    assert L.slots_per_group == pool and L.groups == 4
    idx = pr.idx.reshape(-1, K).long()
    assert bool((idx[:, 1:] > idx[:, :-1]).all()) and int(idx.min()) >= 0 and int(idx.max()) < D
    assert pr.x.shape == (c["B"], D) and pr.x.dtype == c["x_dtype"]
    assert pr.dy.shape == (c["B"], 4)
    if c["indices"] == "window256":
        per_pool = idx.reshape(4, -1)
        assert bool(((per_pool.max(1).values - per_pool.min(1).values) < 256).all())
    if name != "C5":
        assert abs(float(pr.w.std()) - 1 / math.sqrt(K)) < 0.02
    assert pr.b.abs().max() == 0


def test_c5_keeps_top16_of_64_candidates():
    """Brute force: re-derive the kept support of a few neurons from their 64 candidates."""
    from granulelayer_amd.synthetic import _top_k_of_candidates

    gen = torch.Generator().manual_seed(11)
    cand = torch.sort(torch.randperm(4096, generator=gen)[:64]).values[None, :].repeat(3, 1)
    wenv = torch.randn(3, 64, generator=gen) / 4
    # 15 candidates at 1.0, two at 0.9 competing for the last slot: the lower position (5) wins
    wenv[1] = 0.01 * torch.randn(64, generator=gen)
    wenv[1, :5] = 1.0
    wenv[1, 6:9] = 1.0
    wenv[1, 10:17] = 1.0
    wenv[1, 5] = wenv[1, 9] = -0.9
    ki, kw = _top_k_of_candidates(cand, wenv, 16)
    for r in range(3):
        pairs = sorted(((-abs(float(wenv[r, j])), j) for j in range(64)))[:16]
        keep = sorted(int(cand[r, j]) for _, j in pairs)
        assert ki[r].tolist() == keep
        assert all(float(kw[r, i]) == float(wenv[r, (cand[r] == ki[r, i]).nonzero()[0, 0]]) for i in range(16))
    assert int(cand[1, 5]) in ki[1].tolist() and int(cand[1, 9]) not in ki[1].tolist()


def test_state_dict_formats():
    """Checkpoint formats (layer.py:82-88, 133-142): the state-dict keys are the reference's, int16
    indices of a reference checkpoint are widened on load, and a checkpoint that carries an
    input-supergroup plan (`sg_plan`) is refused, since this layer has no connectivity."""
    src = SparsePoolingLayer(64, 3000, 8, shared_neurons=None, pooling="mean", dtype=torch.float32, seed=4)
    sd = src.state_dict()
    assert set(sd) == {"indices", "weight", "bias"}
    dst = SparsePoolingLayer(64, 3000, 8, shared_neurons=None, pooling="mean", dtype=torch.float32, seed=5)
    dst.load_state_dict({**sd, "indices": sd["indices"].to(torch.int16)})
    assert dst.indices.dtype == torch.int32 and torch.equal(dst.indices, sd["indices"])
    assert torch.equal(dst.weight, src.weight) and torch.equal(dst.bias, src.bias)
    plan = torch.frombuffer(bytearray(b'{"kind": "supergroups"}'), dtype=torch.uint8).clone()
    with pytest.raises(ValueError, match="supergroup"):
        dst.load_state_dict({**sd, "sg_plan": plan})


def test_save_winners_over_the_checkpoint_budget_falls_back_to_minimal_stats():
    """save_winners keeps B x U x k int32 ids; above 2 GiB the policy resolves to minimal_stats and
    last_info says why (sparse_pooling/autograd.py:45-56); the recompute chunk keeps one chunk's ids
    within 512 MiB (autograd.py:335)."""
    from types import SimpleNamespace

    from granulelayer_amd.autograd import CHECKPOINT_BUDGET, RECOMPUTE_CHUNK_BYTES, fit_policy, recompute_chunk

    def rt(kind, U, **kw):
        return SimpleNamespace(level=LevelSpec(kind, **kw), units=SimpleNamespace(U=U), last_info={})

    r = rt("topk_mean", 98_304, k=8)
    assert 1024 * 98_304 * 8 * 4 > CHECKPOINT_BUDGET
    assert fit_policy(r, "save_winners", 1024) == "minimal_stats"
    assert "GiB of ids" in r.last_info["policy_fallback"]
    assert fit_policy(r, "save_winners", 256) == "save_winners"  # 0.8 GB fits
    assert "policy_fallback" not in r.last_info
    r = rt("max", 98_304)
    assert fit_policy(r, "save_winners", 5461) == "save_winners"  # 2.15e9 bytes > 2 GiB only from 5462
    assert fit_policy(r, "save_winners", 5462) == "minimal_stats"
    assert fit_policy(rt("mean", 98_304), "minimal_stats", 10**6) == "minimal_stats"
    c = recompute_chunk(rt("topk_mean", 98_304, k=8))
    assert c % 32 == 0 and c * 98_304 * 8 * 4 <= RECOMPUTE_CHUNK_BYTES
    assert recompute_chunk(rt("topk_mean", 10**7, k=64)) == 32  # never below 32 tokens


def test_seeded_init_equals_the_reference_bit_for_bit():
    """init_parameters(layout, seed=s) reproduces the reference's parameters exactly: the same
    indices (widened from the reference's int16), weights and bias, for ragged layouts, a bias std,
    chunked generation and bf16 parameters (fixture written by tests/golden/make_init_golden.py from
    sparse_pooling/layout.py:191-251)."""
    from pathlib import Path

    path = Path(__file__).resolve().parent / "golden" / "init_reference.npz"
    with np.load(path) as z:
        d = {k: z[k] for k in z.files}
    names = sorted({k.split("/")[0] for k in d})
    assert len(names) == 4
    for name in names:
        D, H, G, seed, chunk = (int(v) for v in d[f"{name}/shape"])
        dtype = getattr(torch, str(d[f"{name}/dtype"]))
        L = SparseLayout(D, H, G, 8, 8, False)
        idx, w, b = init_parameters(L, "cpu", dtype=dtype, seed=seed, bias_std=float(d[f"{name}/bias_std"]),
                                    chunk_records=chunk)
        assert L.padding_fraction() > 0, name
        assert np.array_equal(idx.numpy(), d[f"{name}/idx"].astype(np.int32)), f"{name}: indices"
        assert np.array_equal(w.float().numpy(), d[f"{name}/w"]), f"{name}: weights"
        assert np.array_equal(b.float().numpy(), d[f"{name}/b"]), f"{name}: bias"
        assert w.dtype == dtype and b.dtype == dtype and idx.dtype == torch.int32
