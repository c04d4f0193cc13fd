"""Semantic two-level pooling on the CPU: the float64 oracle (oracle/semantic.py) pinned by
finite differences and by the reference's own identities (sparse_pooling/tests/
test_hierarchical_pooling.py:78-131), plus the host logic (units, configuration, parameters)."""
import warnings

import numpy as np
import pytest
import torch

from conftest import assert_close, rel_err
from granulelayer_amd import LevelSpec, PoolingConfig, SparsePoolingLayer
from granulelayer_amd.autograd import make_units
from granulelayer_amd.layout import SparseLayout
from oracle import oracle as O
from oracle import semantic as SO

# (level 1, level 2) pairs of the reference's semantic tests (test_hierarchical_pooling.py:66-76,
# test_backward.py:64-71)
PAIRS = [
    (dict(type="max", neurons_per_shard=256, out_activation="identity"), dict(type="mean")),
    (dict(type="mean", neurons_per_shard=256), dict(type="max")),
    (dict(type="topk_mean", k=4, neurons_per_shard=256), dict(type="logmeanexp", temperature=0.5)),
    (dict(type="max", neurons_per_shard=256, transform="affine"), dict(type="max")),
    (dict(type="topk_mean", k=4, neurons_per_shard=256, transform="gate"), dict(type="weighted_sum")),
    (dict(type="mean", neurons_per_shard=256), dict(type="logmeanexp", temperature=1.0)),
    (dict(type="logmeanexp", temperature=0.5, neurons_per_shard=256), dict(type="mean", activation="identity")),
    (dict(type="mean", neurons_per_shard=512), dict(type="weighted_sum")),
    (dict(type="mean", neurons_per_shard=64, transform="activation", transform_activation="gelu"),
     dict(type="power_mean", p=3.0, activation="relu")),
    (dict(type="sum", neurons_per_shard=64, out_activation="gelu"), dict(type="softmax_weighted", beta=2.0)),
    (dict(type="mean", neurons_per_shard=64), dict(type="topk_mean", k=2, out_activation="relu")),
    (dict(type="mean", neurons_per_shard=64, transform="affine", transform_activation="identity"),
     dict(type="sum", activation="relu")),
]


def _specs(l1, l2):
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        cfg = PoolingConfig([LevelSpec(**l1), LevelSpec(**l2)])
    return cfg.levels


def _tparams(rng, l1, l2, G, S):
    tp = {}
    if l1.transform in ("affine", "gate"):
        tp["alpha"] = 1.0 + 0.3 * rng.standard_normal((G, S))
        tp["beta"] = 0.3 * rng.standard_normal((G, S))
    if l2.type == "weighted_sum":
        tp["v"] = 1.0 / S + 0.3 * rng.standard_normal((G, S))
    return tp


@pytest.mark.parametrize("l1,l2", PAIRS, ids=lambda d: d["type"])
def test_level2_backward_matches_finite_differences(l1, l2):
    l1, l2 = _specs(l1, l2)
    rng = np.random.default_rng(3)
    B, G, S = 3, 4, 5
    F = rng.standard_normal((B, G, S))
    tp = _tparams(rng, l1, l2, G, S)
    dy = rng.standard_normal((B, G))
    dF, dt = SO.level2_backward(F, l1, l2, tp, dy)
    f = lambda F_, tp_: float((SO.level2_forward(F_, l1, l2, tp_) * dy).sum())  # noqa: E731
    h = 1e-6
    num = np.zeros_like(F)
    for i in np.ndindex(F.shape):
        Fp, Fm = F.copy(), F.copy()
        Fp[i] += h
        Fm[i] -= h
        num[i] = (f(Fp, tp) - f(Fm, tp)) / (2 * h)
    assert_close(dF, num, rtol=1e-5, atol=1e-7, what="dF")
    for name, g in dt.items():
        numt = np.zeros_like(tp[name])
        for i in np.ndindex(numt.shape):
            tpp = {k: v.copy() for k, v in tp.items()}
            tpm = {k: v.copy() for k, v in tp.items()}
            tpp[name][i] += h
            tpm[name][i] -= h
            numt[i] = (f(F, tpp) - f(F, tpm)) / (2 * h)
        assert_close(g, numt, rtol=1e-5, atol=1e-7, what=f"d{name}")
    assert set(dt) == set(tp)


def test_level2_special_cases():
    rng = np.random.default_rng(4)
    B, G, S = 4, 3, 6
    F = rng.standard_normal((B, G, S))
    l1, l2 = _specs(dict(type="mean", neurons_per_shard=32), dict(type="weighted_sum"))
    _, mean = _specs(dict(type="mean", neurons_per_shard=32), dict(type="mean", activation="identity"))
    ws = SO.level2_forward(F, l1, l2, {"v": np.full((G, S), 1.0 / S)})
    assert_close(ws, SO.level2_forward(F, l1, mean, {}), rtol=1e-12, atol=1e-12, what="v = 1/S is the mean")
    assert_close(ws, F.mean(-1), rtol=1e-12, atol=1e-12, what="mean")
    # one shard: the level-2 pool of a single feature is that feature's activation
    for l2d in (dict(type="max"), dict(type="logmeanexp", temperature=0.7), dict(type="power_mean", p=2.5),
                dict(type="softmax_weighted", beta=3.0), dict(type="topk_mean", k=4)):
        _, l2s = _specs(dict(type="mean", neurons_per_shard=32), l2d)
        y = SO.level2_forward(np.abs(F[..., :1]), l1, l2s, {})
        assert_close(y, np.abs(F[..., 0]), rtol=1e-12, atol=1e-12, what=l2d["type"])


def _layer_problem(seed, B, D, H, G, K=8):
    L = SparseLayout(D, H, G, K, 8, False)
    rng = np.random.default_rng(seed)
    counts, _, S = O.partition(H, G)
    assert S == L.slots_per_group
    idx = np.zeros((G * S, K), np.int32)
    w = np.zeros((G * S, K), np.float32)
    b = np.zeros(G * S, np.float32)
    for g in range(G):
        for s in range(counts[g]):
            n = g * S + s
            idx[n] = np.sort(rng.choice(D, K, replace=False))
            w[n] = rng.standard_normal(K).astype(np.float32) / np.sqrt(K)
            b[n] = rng.standard_normal() * 0.3
    x = rng.standard_normal((B, D)).astype(np.float32)
    return x, idx, w, b, counts, S


@pytest.mark.parametrize("H,G,nps", [(3001, 8, 256), (8 * 600, 8, 256), (2048, 4, 128), (700, 3, 32)])
def test_sum_of_shard_sums_is_the_flat_sum(H, G, nps):
    """Sum -> Sum with identity activations is the flat sum over the group whatever the shard sizes:
    pins the shard boundaries (every valid neuron in exactly one shard) and the gradient scatter."""
    x, idx, w, b, counts, S = _layer_problem(1, 5, 64, H, G)
    l1, l2 = _specs(dict(type="sum", activation="identity", neurons_per_shard=nps),
                    dict(type="sum", activation="identity"))
    y, F, pre, _ = SO.forward_two_level(x, idx, w, b, counts, S, l1, l2, {})
    flat = O.forward(x, idx, w, b, counts, S, act="identity", pool="sum")
    assert_close(y, flat, rtol=1e-12, atol=1e-10, what="y")
    dy = np.random.default_rng(2).standard_normal(y.shape).astype(np.float32)
    dW, db, dX, dt = SO.backward_two_level(x, idx, w, b, counts, S, l1, l2, {}, dy)
    fW, fb, fX = O.backward(x, idx, w, b, counts, S, dy, act="identity", pool="sum")
    assert_close(dW, fW, rtol=1e-12, atol=1e-12, what="dW")
    assert_close(db, fb, rtol=1e-12, atol=1e-12, what="db")
    assert_close(dX, fX, rtol=1e-12, atol=1e-10, what="dX")
    assert dt == {}


def test_mean_of_shard_means_is_the_flat_mean_only_with_full_shards():
    """test_hierarchical_pooling.py:104-115: equal with full shards, a different model with a partial one."""
    l1, l2 = _specs(dict(type="mean", activation="identity", neurons_per_shard=256),
                    dict(type="mean", activation="identity"))
    x, idx, w, b, counts, S = _layer_problem(2, 4, 64, 8 * 512, 8)  # every group 512 = 2 full shards
    y, *_ = SO.forward_two_level(x, idx, w, b, counts, S, l1, l2, {})
    assert_close(y, O.forward(x, idx, w, b, counts, S, act="identity", pool="mean"), rtol=1e-12, atol=1e-12,
                 what="full shards")
    x, idx, w, b, counts, S = _layer_problem(2, 4, 64, 8 * 600, 8)  # 256 + 256 + 88
    y, *_ = SO.forward_two_level(x, idx, w, b, counts, S, l1, l2, {})
    assert not np.allclose(y, O.forward(x, idx, w, b, counts, S, act="identity", pool="mean"), atol=1e-4)


def test_max_of_shard_maxima_is_the_flat_maximum():
    """test_hierarchical_pooling.py:97-101: Max -> Max without a non-monotone transform is global Max."""
    l1, l2 = _specs(dict(type="max", neurons_per_shard=256), dict(type="max"))
    x, idx, w, b, counts, S = _layer_problem(3, 6, 64, 3000, 8)
    y, *_ = SO.forward_two_level(x, idx, w, b, counts, S, l1, l2, {})
    pre, _, _ = O.forward_max(x, idx, w, b, counts, S, act=l1.activation)
    assert_close(y, np.maximum(pre, 0.0), rtol=1e-12, atol=1e-12, what="Max -> Max")


def test_two_level_backward_matches_finite_differences_through_both_levels():
    """dX of the whole two-level model against central differences of its float64 forward (smooth
    operators at both levels, so the model is differentiable everywhere)."""
    l1, l2 = _specs(dict(type="logmeanexp", temperature=0.5, neurons_per_shard=32, transform="gate"),
                    dict(type="softmax_weighted", beta=1.5))
    x, idx, w, b, counts, S = _layer_problem(5, 2, 16, 200, 3)
    rng = np.random.default_rng(6)
    Sh, _ = SO.shard_units(counts, 32)
    tp = _tparams(rng, l1, l2, 3, Sh)
    dy = rng.standard_normal((2, 3)).astype(np.float32)
    _, _, dX, _ = SO.backward_two_level(x, idx, w, b, counts, S, l1, l2, tp, dy)
    f = lambda xx: float((SO.forward_two_level(xx, idx, w, b, counts, S, l1, l2, tp)[0] * dy).sum())  # noqa: E731
    h = 1e-2  # x is rounded to fp32 by the C oracle: a wide step keeps the rounding small
    num = np.zeros_like(dX)
    for i in np.ndindex(x.shape):
        xp, xm = x.astype(np.float64).copy(), x.astype(np.float64).copy()
        xp[i] += h
        xm[i] -= h
        num[i] = (f(xp) - f(xm)) / (2 * h)
    assert rel_err(dX, num) < 1e-3


def test_units_and_configuration():
    L = SparseLayout(64, 3000, 8, 8, 8, False)
    u = make_units(L, 256, "cpu")
    assert u.S == 2 and u.nps == 256 and u.U == 16
    assert u.counts.tolist() == [256.0, 119.0] * 8
    assert make_units(L, None, "cpu").U == 8
    with pytest.raises(ValueError, match="multiple of 4"):
        make_units(L, 100, "cpu")
    with pytest.raises(ValueError, match="empty"):  # counts 129, 128, 128: 3 shards of 64, the last empty for two
        make_units(SparseLayout(64, 385, 3, 8, 8, False), 64, "cpu")
    assert LevelSpec("mean", neurons_per_shard=256).hip_reason() == ""
    assert LevelSpec("mean", neurons_per_shard=100).hip_reason()


def test_layer_two_level_parameters_on_cpu():
    lay = SparsePoolingLayer(64, 3000, 8, fan_in=8, shared_neurons=None,
                             pooling={"levels": [dict(type="max", neurons_per_shard=256, transform="affine"),
                                                 dict(type="weighted_sum")]}, dtype=torch.float32)
    assert lay.num_shards == 2
    assert lay._tnames == ["alpha", "beta", "v"]
    assert torch.equal(lay.t_alpha, torch.ones(8, 2)) and torch.equal(lay.t_beta, torch.zeros(8, 2))
    assert torch.equal(lay.t_v, torch.full((8, 2), 0.5))
    sd = lay.state_dict()
    assert {"t_alpha", "t_beta", "t_v", "weight", "bias", "indices"} <= set(sd)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        lay(torch.randn(2, 64))


def _mirror_pool_base(g, S, sps, gs):
    # the kernels' neuron address of pool g's first slot (gl_common.h pool_base / pool_ext)
    if sps <= 1:
        return g * S, S
    return (g // sps) * gs + (g % sps) * S, min(S, gs - (g % sps) * S)


@pytest.mark.parametrize("D,H,G,nps", [(64, 3000, 8, 256), (64, 3000, 8, 512), (64, 3000, 8, 64), (64, 3000, 8, 96),
                                       (1024, 20011, 16, 256), (256, 12000, 12, 96), (512, 9000, 6, 512),
                                       (512, 9000, 6, 160), (2048, 65536, 8, 4096), (64, 3000, 8, 384),
                                       (64, 2048, 8, 256), (64, 3000, 8, None)])
def test_pool_geometry_of_the_launches_stays_inside_the_layout(D, H, G, nps):
    """The geometry HipBackend hands the kernels (pools, slots per pool, sps, gs, counts) for every
    shard configuration the GPU tests run: each of the 64 * cpg slots of every pool addresses a
    neuron of the layout (padded slots clamp to the pool's last slot inside its group), and each
    valid slot a neuron of its own group, every valid neuron exactly once."""
    from types import SimpleNamespace

    from granulelayer_amd.backend import HipBackend

    L = SparseLayout(D, H, G, 8, 8, False)
    units = make_units(L, nps, "cpu")
    rt = SimpleNamespace(layout=L, units=units, counts_i32=L.counts_tensor("cpu"),
                         unit_counts_i32=units.counts.to(torch.int32))
    U, S, sps, gs, counts = HipBackend._pools(rt)
    counts = counts.numpy()
    rows = L.groups * L.slots_per_group
    group_counts = L.counts_tensor("cpu").numpy()
    seen = np.zeros(rows, np.int64)
    span = -(-S // 256) * 256  # slots of the pool's chunks (64 lanes x 4 neurons)
    for g in range(U):
        base, ext = _mirror_pool_base(g, S, sps, gs)
        assert 1 <= counts[g] <= ext
        s = np.arange(span)
        n = base + np.minimum(s, ext - 1)
        assert n.min() >= 0 and n.max() < rows
        v = n[s < counts[g]]
        grp = v // L.slots_per_group
        assert (grp == (g // sps if sps > 1 else g)).all()
        assert (v % L.slots_per_group < group_counts[grp]).all()
        seen[v] += 1
    valid = (np.arange(L.slots_per_group)[None, :] < group_counts[:, None]).reshape(-1)
    assert (seen[valid] == 1).all() and (seen[~valid] == 0).all()
