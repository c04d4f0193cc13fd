"""Semantic two-level pooling on the GPU: level-1 shards on the HIP kernels, level 2 in torch,
against the float64 oracle (oracle/semantic.py) on identical seeded inputs.

* layer level: y, dX, dW, db and the transform / weighted-sum parameters' gradients of the
  reference's semantic cases (sparse_pooling/tests/test_hierarchical_pooling.py:66-101,
  test_backward.py:64-71) under level1_checkpoint "save" and "recompute", with the reference's
  bar rel_err < 2e-5 (test_hierarchical_pooling.py:96);
* kernel level: the shards' pooled values and selected slots (Level1Runtime with
  neurons_per_shard) elementwise against the oracle's error scale, on ragged groups whose last
  shard ends inside the group, and dW / db / dX of a given g_pre;
* Max -> Max equals the flat maximum (test_hierarchical_pooling.py:97-101)."""
import warnings

import numpy as np
import pytest
import torch

from conftest import assert_parity, gpu_available, rel_err

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

from granulelayer_amd import LevelSpec, PhysicalPlan, PoolingConfig, SparsePoolingLayer  # noqa: E402
from granulelayer_amd.autograd import Level1Runtime  # noqa: E402
from granulelayer_amd.layout import SparseLayout, init_parameters  # noqa: E402
from oracle import oracle as O  # noqa: E402
from oracle import semantic as SO  # noqa: E402

DEV = "cuda"

SEMANTIC = [
    (dict(type="max", neurons_per_shard=256, out_activation="identity"), dict(type="mean")),
    (dict(type="mean", neurons_per_shard=256), dict(type="max")),
    (dict(type="topk_mean", k=4, neurons_per_shard=256), dict(type="logmeanexp", temperature=0.5)),
    (dict(type="max", neurons_per_shard=256, transform="affine"), dict(type="max")),
    (dict(type="topk_mean", k=4, neurons_per_shard=256, transform="gate"), dict(type="weighted_sum")),
    (dict(type="mean", neurons_per_shard=256), dict(type="logmeanexp", temperature=1.0)),
    (dict(type="logmeanexp", temperature=0.5, neurons_per_shard=256), dict(type="mean", activation="identity")),
    (dict(type="mean", neurons_per_shard=512), dict(type="weighted_sum")),
    (dict(type="logmeanexp", temperature=0.5, neurons_per_shard=512, transform="gate"), dict(type="max")),
    (dict(type="softmax_weighted", beta=2.0, neurons_per_shard=64, out_activation="gelu"),
     dict(type="power_mean", p=3.0, activation="relu")),
    (dict(type="sum", neurons_per_shard=96, transform="activation", transform_activation="gelu"),
     dict(type="topk_mean", k=2)),
]


def _cfg(l1, l2, **kw):
    return {"levels": [l1, l2], **kw}


def _layer(D, H, G, cfg, policy="auto", seed=1):
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        lay = SparsePoolingLayer(D, H, G, fan_in=8, shared_neurons=None, pooling=cfg, checkpoint_policy=policy,
                                 dtype=torch.float32, device=DEV, seed=seed, bias_std=0.2)
    with torch.no_grad():  # non-trivial learned transforms, as the reference's test makes them
        gen = torch.Generator().manual_seed(seed + 7)
        for n in lay._tnames:
            t = getattr(lay, "t_" + n)
            t.add_((0.3 * torch.randn(t.shape, generator=gen)).to(DEV))
    return lay


def _oracle_two_level(lay, x, dy):
    L = lay.layout
    K = L.fan_in
    l1, l2 = lay.cfg.levels
    idx = lay.indices.cpu().reshape(-1, K).numpy()
    w = lay.weight.detach().cpu().reshape(-1, K).numpy()
    b = lay.bias.detach().cpu().reshape(-1).numpy()
    counts = L.counts_tensor("cpu").numpy()
    tp = {n: getattr(lay, "t_" + n).detach().cpu().double().numpy() for n in lay._tnames}
    xn = x.detach().cpu().float().numpy()
    y, F, pre, mag = SO.forward_two_level(xn, idx, w, b, counts, L.slots_per_group, l1, l2, tp)
    dW, db, dX, dt = SO.backward_two_level(xn, idx, w, b, counts, L.slots_per_group, l1, l2, tp,
                                           dy.detach().cpu().numpy())
    return y, dW, db, dX, dt


@pytest.mark.parametrize("l1,l2", SEMANTIC, ids=lambda d: d["type"] + str(d.get("neurons_per_shard", "")))
@pytest.mark.parametrize("ckpt", ["save", "recompute"])
def test_two_level_layer_matches_oracle(l1, l2, ckpt):
    lay = _layer(64, 3000, 8, _cfg(l1, l2, level1_checkpoint=ckpt))
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(32, 64, generator=gen).to(DEV).requires_grad_(True)
    dy = torch.randn(32, 8, generator=gen).to(DEV)
    y = lay(x)
    # the backward reruns level 1 once under "recompute" (with the selected slots a max / top-k
    # level 1 needs) and never under "save"
    rt, calls = lay._runtime(), []
    fwd = rt.forward
    rt.forward = lambda *a, **k: (calls.append(k.get("track_ids", False)), fwd(*a, **k))[1]
    (y * dy).sum().backward()
    del rt.forward
    assert len(calls) == (1 if ckpt == "recompute" else 0), calls
    wy, wdW, wdb, wdX, wdt = _oracle_two_level(lay, x, dy)
    K = lay.layout.fan_in
    got = {"y": y.detach(), "dX": x.grad, "dW": lay.weight.grad.reshape(-1, K), "db": lay.bias.grad.reshape(-1)}
    want = {"y": wy, "dX": wdX, "dW": wdW, "db": wdb}
    for n in lay._tnames:
        got["d" + n] = getattr(lay, "t_" + n).grad
        want["d" + n] = wdt[n]
    for k in got:
        e = rel_err(got[k].cpu().numpy(), want[k])
        assert e < 2e-5, f"{k}: rel_err {e:.2e}"
    info = lay.last_info
    assert info["forward_backend"] == "hip" and info["backward_backend"] == "hip"
    if ckpt == "recompute":
        assert info["checkpoint_bytes"] == 0


@pytest.mark.parametrize("policy", ["minimal_stats", "save_winners", "recompute_stats"])
def test_two_level_policies_agree_bitwise(policy):
    """The checkpoint policy changes what is saved, not the result: every policy gives the bits of
    save_winners (max level 1, whose backward needs the winners)."""
    cfg = _cfg(dict(type="max", neurons_per_shard=256, transform="affine"), dict(type="max"))
    outs = []
    for pol in ("save_winners", policy):
        lay = _layer(64, 3000, 8, cfg, policy=pol)
        gen = torch.Generator().manual_seed(3)
        x = torch.randn(16, 64, generator=gen).to(DEV).requires_grad_(True)
        dy = torch.randn(16, 8, generator=gen).to(DEV)
        (lay(x) * dy).sum().backward()
        outs.append((x.grad.clone(), lay.weight.grad.clone(), lay.t_alpha.grad.clone()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


# (D, H, G, nps, pool, B, x dtype): ragged groups whose last shard ends inside the group
KERNEL_CASES = [
    (1024, 20011, 16, 256, "mean", 64, torch.bfloat16),
    (1024, 20011, 16, 256, "max", 70, torch.float32),
    (256, 12000, 12, 96, "topk_mean", 40, torch.float32),
    (512, 9000, 6, 512, "logmeanexp", 33, torch.float32),
    (512, 9000, 6, 160, "softmax_weighted", 33, torch.float32),
    (2048, 65536, 8, 4096, "sum", 130, torch.float32),
]


@pytest.mark.parametrize("case", KERNEL_CASES, ids=lambda c: f"{c[4]}-nps{c[3]}-D{c[0]}")
def test_shard_kernels_match_oracle(case):
    D, H, G, nps, pool, B, xdt = case
    L = SparseLayout(D, H, G, 8, 8, False)
    idx, w, b = init_parameters(L, "cpu", torch.float32, seed=5, bias_std=0.3)
    lv = LevelSpec(pool, k=4, temperature=0.7, beta=1.5, neurons_per_shard=nps,
                   activation="identity" if pool in ("max", "topk_mean") else "relu")
    rt = Level1Runtime(L, idx.to(DEV), lv, PhysicalPlan(), nps)
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(B, D, generator=gen).to(xdt)
    S = L.slots_per_group
    out = rt.forward(x.to(DEV), w.to(DEV), b.to(DEV), track_ids=pool in ("max", "topk_mean"))
    U = rt.units.U
    assert out["pre"].shape == (B, U) and U == G * rt.units.S
    fi, fw, fb = idx.reshape(-1, 8).numpy(), w.reshape(-1, 8).numpy(), b.reshape(-1).numpy()
    counts = L.counts_tensor("cpu").numpy()
    xn = x.float().numpy()
    pre, mag, sel = SO.level1_forward(xn, fi, fw, fb, counts, S, nps, lv)
    assert_parity(out["pre"].cpu().numpy(), pre, mag + np.abs(pre), what="shard pre")
    if pool == "max":
        agree = (out["winner"].cpu().numpy() == sel).mean()
        assert agree > 0.999, agree
    g_pre = torch.randn(B, U, generator=gen)
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(x.to(DEV), w.to(DEV), b.to(DEV), g_pre.to(DEV), out, "minimal_stats", dw, db).cpu().numpy()
    wdW, wdb, wdX = SO.level1_backward(xn, fi, fw, fb, counts, S, nps, lv, g_pre.numpy())
    for k, (a, e) in {"dX": (dx, wdX), "dW": (dw.cpu().numpy().reshape(-1, 8), wdW),
                      "db": (db.cpu().numpy().reshape(-1), wdb)}.items():
        assert rel_err(a, e) < 2e-5, f"{pool} {k}: rel_err {rel_err(a, e):.2e}"
    # padded slots and every slot past a group's count keep a zero gradient
    valid = (np.arange(S)[None, :] < counts[:, None]).reshape(-1)
    assert not dw.cpu().numpy().reshape(-1, 8)[~valid].any()


def test_max_of_shard_maxima_is_the_flat_maximum_on_the_gpu():
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        lay = _layer(64, 3000, 8, _cfg(dict(type="max", neurons_per_shard=256), dict(type="max")))
        flat = SparsePoolingLayer(64, 3000, 8, fan_in=8, shared_neurons=None, pooling="max", dtype=torch.float32,
                                  device=DEV, seed=1, bias_std=0.2)
    x = torch.randn(16, 64, generator=torch.Generator().manual_seed(2)).to(DEV)
    assert torch.equal(lay(x).detach(), flat(x).detach())
