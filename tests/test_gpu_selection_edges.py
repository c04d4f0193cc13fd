"""Selection pooling edge cases on the GPU against the oracle: NaN candidates in the top-k merge,
and the fixed-point dX of the selection backward when the terms of different inputs differ by many
orders of magnitude."""
import numpy as np
import pytest
import torch

from conftest import assert_parity, gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

from granulelayer_amd import LevelSpec, PhysicalPlan, SparseLayout, init_parameters  # noqa: E402
from granulelayer_amd.autograd import Level1Runtime  # noqa: E402
from oracle import oracle as O  # noqa: E402

DEV = "cuda"


def _layer(D, H, G, B, seed, disjoint=False):
    L = SparseLayout(D, H, G, 8, 8, False)
    idx, w, b = init_parameters(L, "cpu", torch.float32, seed=seed, bias_std=0.2)
    if disjoint:  # pool g reads only inputs [g * D / G, (g + 1) * D / G)
        from granulelayer_amd.layout import sample_distinct

        S, width = L.slots_per_group, D // G
        gen = torch.Generator().manual_seed(seed + 3)
        rec = sample_distinct(G * S, width, 8, gen, "cpu").to(torch.int32)
        rec += (torch.arange(G * S) // S * width).to(torch.int32)[:, None]
        rec[~L.valid_mask("cpu").reshape(-1)] = 0
        idx = rec.view(L.index_shape)
    gen = torch.Generator().manual_seed(seed + 1000)
    x = torch.randn(B, D, generator=gen)
    dy = torch.randn(B, G, generator=gen)
    return L, idx, w, b, x, dy


def _flat(L, idx, w, b):
    return idx.reshape(-1, 8).numpy(), w.reshape(-1, 8).numpy(), b.reshape(-1).numpy()


@pytest.mark.parametrize("sign", [1.0, -1.0])
@pytest.mark.parametrize("k", [8, 4])
def test_topk_nan_candidate_in_a_later_chunk_is_selected_first(sign, k):
    """A neuron whose z is NaN (of either sign) ranks above every number, as in torch.sort: it is
    the first pick of its pool for every token, wherever its chunk lies; its pool's other k - 1
    picks are the oracle's top-(k - 1) without it, and every other pool's picks are the oracle's."""
    D, H, G, B = 256, 4 * 1024, 4, 23
    L, idx, w, b, x, _ = _layer(D, H, G, B, seed=11)
    S = L.slots_per_group
    slot = 2 * 256 + 37  # in the pool's third chunk of 256 slots
    n = 1 * S + slot
    bf = b.clone()
    bf.view(-1)[n] = sign * float("nan")
    rt = Level1Runtime(L, idx.to(DEV), LevelSpec("topk_mean", activation="identity", k=k), PhysicalPlan())
    out = rt.forward(x.to(DEV), w.to(DEV), bf.to(DEV), track_ids=True)
    got = out["topk_slot"].cpu().numpy()
    pre = out["pre"].cpu().numpy()
    assert (got[:, 1, 0] == slot).all(), "the NaN neuron is every token's first pick in pool 1"
    assert np.isnan(pre[:, 1]).all() and not np.isnan(np.delete(pre, 1, axis=1)).any()
    counts = L.counts_tensor("cpu").numpy()
    # pool 1 without the NaN neuron (its z pushed to -100, far below every other: never selected),
    # k - 1 picks; the oracle's margin is relative to the pool's largest |term|, which stays ~100
    bx = b.clone()
    bx.view(-1)[n] = -100.0
    fi, fw, fb = _flat(L, idx, w, bx)
    _, want1, gap1 = O.forward_topk(x.numpy(), fi, fw, fb, counts, S, k - 1)
    clear1 = gap1[:, 1] > 2e-6
    assert clear1.mean() > 0.9
    assert (np.sort(got[:, 1, 1:], -1)[clear1] == np.sort(want1[:, 1], -1)[clear1]).all()
    # the other pools are untouched
    fi, fw, fb = _flat(L, idx, w, b)
    _, want, gap = O.forward_topk(x.numpy(), fi, fw, fb, counts, S, k)
    others = [0, 2, 3]
    clear = gap[:, others] > 2e-6
    assert clear.mean() > 0.95
    assert (np.sort(got[:, others], -1)[clear] == np.sort(want[:, others], -1)[clear]).all()


@pytest.mark.parametrize("pool,k", [("max", 1), ("topk_mean", 8)])
def test_selection_dx_keeps_relative_precision_of_small_inputs(pool, k):
    """Pools read disjoint input ranges, and dY of half the pools is 1e-12 of the others, so half
    the inputs receive terms ~12 orders below the token's largest term.  The fixed-point dX scales
    each input by its own largest term: every dX entry meets the fp32 bar against the oracle's
    float64 sum relative to its own terms' magnitude."""
    D, H, G, B = 2048, 8 * 1024, 8, 40
    L, idx, w, b, x, dy = _layer(D, H, G, B, seed=12, disjoint=True)
    dy[:, G // 2:] *= 1e-12
    spec = LevelSpec(pool, activation="relu", k=k) if pool == "topk_mean" else LevelSpec(pool, activation="relu")
    rt = Level1Runtime(L, idx.to(DEV), spec, PhysicalPlan())
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    st = rt.forward(xd, wd, bd, track_ids=True)
    key = "winner" if pool == "max" else "topk_slot"
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(xd, wd, bd, dy.to(DEV), st, "save_winners", dw, db).cpu().numpy()
    fi, fw, fb = _flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_events(x.numpy(), fi, fw, fb, counts, L.slots_per_group, dy.numpy(),
                                                    st[key].cpu().numpy(), "relu", topk=pool == "topk_mean")
    small = slice(D // 2, D)
    assert np.abs(wdX[:, small]).max() < 1e-9 * np.abs(wdX[:, :D // 2]).max()
    assert_parity(dx[:, small], wdX[:, small], mX[:, small], what=f"{pool} dX of the small inputs")
    assert_parity(dx, wdX, mX, what=f"{pool} dX")
    assert_parity(dw.cpu().numpy().reshape(-1, 8), wdW, mW, what=f"{pool} dW")
