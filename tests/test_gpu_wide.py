"""Input widths past one LDS token tile (D > 10,112, up to the reference's 32,767,
sparse_pooling/layout.py:57-58): the forward, dW and smooth recompute kernels gather X from the
token tiles in global memory and the selection events' dX walks the inputs in blocks.  Forward and
backward of every pooling kind against the float64 oracle on identical seeded inputs (fp32 bar of
conftest.assert_parity), K = 8 and 16, bf16 X, window staging; the same layer at a narrow D gives
the same bits through the LDS path (the gather source does not change any arithmetic).

Widths 4097..8192 (even) run sum / mean forward and dW over two-token tiles (8-byte slots, one
64-KiB buffer per tile): the same oracle checks, ragged token counts, and the bits of the
four-token path for the same layer."""
import numpy as np
import pytest
import torch

from conftest import assert_parity, gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

from granulelayer_amd import LevelSpec, PhysicalPlan  # noqa: E402
from granulelayer_amd.autograd import Level1Runtime  # noqa: E402
from oracle import oracle as O  # noqa: E402
from test_gpu_parity import flat, make_case, make_window_case  # noqa: E402

DEV = "cuda"

WIDE = [
    # D, H, G, K, B, x dtype
    (16384, 12000, 12, 8, 37, torch.float32),
    (32767, 9000, 9, 8, 70, torch.bfloat16),
    (20000, 6000, 6, 16, 33, torch.float32),
]
TWO_TOKEN = [
    # D, H, G, K, B, x dtype: two-token tiles (even D in 4097..8192); 5001 is odd (one 16-byte-slot tile)
    (8192, 12000, 12, 8, 37, torch.bfloat16),
    (6000, 20011, 16, 8, 130, torch.float32),
    (4098, 7000, 7, 16, 66, torch.float32),
    (8190, 9000, 9, 8, 2, torch.float32),
    (5001, 8000, 8, 8, 33, torch.float32),
]
_ids = lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}{str(c[5])[6:]}"  # noqa: E731


def _rt(L, idx, spec):
    return Level1Runtime(L, idx.to(DEV), spec, PhysicalPlan())


@pytest.mark.parametrize("case", WIDE + TWO_TOKEN, ids=_ids)
@pytest.mark.parametrize("pool,act", [("mean", "relu"), ("sum", "identity")])
def test_wide_sum_and_mean(case, pool, act):
    D, H, G, K, B, xdt = case
    L, idx, w, b, x, dy = make_case(D, H, G, K, B, x_dtype=xdt)
    rt = _rt(L, idx, LevelSpec(pool, activation=act))
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    pre = rt.forward(xd, wd, bd)["pre"].cpu().numpy()
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    xn = x.float().numpy()
    want, mag = O.forward(xn, fi, fw, fb, counts, L.slots_per_group, act, pool, with_mag=True)
    assert_parity(pre, want, mag, what="pre")
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(xd, wd, bd, dy.to(DEV), {}, "minimal_stats", dw, db).cpu().numpy()
    wdW, wdb, wdX, bnd = O.backward(xn, fi, fw, fb, counts, L.slots_per_group, dy.numpy(), act, pool,
                                    with_bounds=True)
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_parity(dx, wdX, mX, uX, what="dX")
    assert_parity(dw.cpu().numpy().reshape(-1, K), wdW, mW, uW, what="dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, ub, what="db")


@pytest.mark.parametrize("case", WIDE[:2], ids=_ids)
@pytest.mark.parametrize("pool", ["max", "topk_mean"])
def test_wide_selection(case, pool):
    """Max and top-8 mean: the forward's values and (where the selection's lead exceeds fp32
    rounding) its slots, and the event backward of the GPU's own selection; D = 32767 runs the
    events' dX in three input blocks."""
    D, H, G, K, B, xdt = case
    L, idx, w, b, x, dy = make_case(D, H, G, K, B, x_dtype=xdt)
    k = 8
    rt = _rt(L, idx, LevelSpec(pool, activation="identity", k=k))
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    out = rt.forward(xd, wd, bd, track_ids=True)
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    xn = x.float().numpy()
    if pool == "max":
        want, sel, gap = O.forward_max(xn, fi, fw, fb, counts, L.slots_per_group, act="identity")
        got_sel = out["winner"].cpu().numpy()
        clear = gap > 2e-6
        assert np.array_equal(got_sel[clear], sel[clear])
    else:
        want, sel, gap = O.forward_topk(xn, fi, fw, fb, counts, L.slots_per_group, k, act="identity")
        got_sel = out["topk_slot"].cpu().numpy()
        clear = gap > 2e-6
        assert np.array_equal(np.sort(got_sel[clear], -1), np.sort(sel[clear], -1))
    np.testing.assert_allclose(out["pre"].cpu().numpy(), want, rtol=1e-5, atol=1e-5)
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(xd, wd, bd, dy.to(DEV), out, "save_winners", dw, db).cpu().numpy()
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_events(xn, fi, fw, fb, counts, L.slots_per_group, dy.numpy(), got_sel,
                                                    act="identity", topk=pool == "topk_mean")
    assert_parity(dx, wdX, mX, what="dX")
    assert_parity(dw.cpu().numpy().reshape(-1, K), wdW, mW, what="dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, what="db")


@pytest.mark.parametrize("case", [WIDE[0], WIDE[2]], ids=_ids)
@pytest.mark.parametrize("pool,param", [("logmeanexp", 0.7), ("softmax_weighted", 1.5)])
def test_wide_smooth(case, pool, param):
    D, H, G, K, B, xdt = case
    L, idx, w, b, x, dy = make_case(D, H, G, K, B, x_dtype=xdt)
    kw = {"logmeanexp": "temperature", "softmax_weighted": "beta"}[pool]
    rt = _rt(L, idx, LevelSpec(pool, activation="relu", **{kw: param}))
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    out = rt.forward(xd, wd, bd)
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    xn = x.float().numpy()
    want, _, mag = O.forward_smooth(xn, fi, fw, fb, counts, L.slots_per_group, pool, param, "relu")
    assert_parity(out["pre"].cpu().numpy(), want, mag, what="pre")
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(xd, wd, bd, dy.to(DEV), out, "minimal_stats", dw, db).cpu().numpy()
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_smooth(xn, fi, fw, fb, counts, L.slots_per_group, dy.numpy(), pool,
                                                    param, "relu")
    assert_parity(dx, wdX, mX, what="dX")
    assert_parity(dw.cpu().numpy().reshape(-1, K), wdW, mW, what="dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, what="db")


def test_wide_window_staging():
    """Narrow pool windows at D = 16384 stage only the windows in LDS (the global gather is not used)."""
    L, idx, w, b, x, dy = make_window_case(16384, 8192, 8, 8, 37, 256)
    rt = _rt(L, idx, LevelSpec("mean", activation="relu"))
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    pre = rt.forward(xd, wd, bd)["pre"].cpu().numpy()
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    want, mag = O.forward(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group, "relu", "mean", with_mag=True)
    assert_parity(pre, want, mag, what="pre")


def test_global_gather_gives_the_bits_of_the_lds_path():
    """One layer's parameters (indices below 4096) run at D = 4096 (LDS tiles) and D = 12288
    (global gathers; X's extra columns unused): pre, dW, db and dX of the shared inputs are
    bit-identical (same edges, same order, same dX unit ranges)."""
    from granulelayer_amd.layout import SparseLayout

    L4, idx, w, b, x4, dy = make_case(4096, 8000, 8, 8, 40, seed=9)
    outs = []
    for D in (4096, 12288):
        L = L4 if D == 4096 else SparseLayout(D, 8000, 8, 8, 8, False)
        x = torch.zeros(40, D)
        x[:, :4096] = x4
        rt = _rt(L, idx, LevelSpec("mean", activation="relu"))
        xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
        pre = rt.forward(xd, wd, bd)["pre"]
        dw = torch.zeros(L.weight_shape, device=DEV)
        db = torch.zeros(L.bias_shape, device=DEV)
        dx = rt.backward(xd, wd, bd, dy.to(DEV), {}, "minimal_stats", dw, db)
        outs.append((pre.cpu(), dw.cpu(), db.cpu(), dx[:, :4096].cpu()))
        if D > 4096:
            assert not dx[:, 4096:].any()
    for a, c in zip(*outs):
        assert torch.equal(a, c)


def test_two_token_tiles_give_the_bits_of_four_token_tiles():
    """One layer's parameters (indices below 4096) at D = 4096 (four-token tiles) and D = 8192
    (two-token tiles; X's extra columns unused): pre, dW, db and dX of the shared inputs are
    bit-identical.  Per token the sums run over the same neurons, edges and lanes in the same
    order; the two-token wave reduction pairs the lanes as the four-token one does."""
    from granulelayer_amd.layout import SparseLayout

    L4, idx, w, b, x4, dy = make_case(4096, 8000, 8, 8, 41, seed=10)
    outs = []
    for D in (4096, 8192):
        L = L4 if D == 4096 else SparseLayout(D, 8000, 8, 8, 8, False)
        x = torch.zeros(41, D)
        x[:, :4096] = x4
        rt = _rt(L, idx, LevelSpec("mean", activation="relu"))
        xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
        pre = rt.forward(xd, wd, bd)["pre"]
        dw = torch.zeros(L.weight_shape, device=DEV)
        db = torch.zeros(L.bias_shape, device=DEV)
        dx = rt.backward(xd, wd, bd, dy.to(DEV), {}, "minimal_stats", dw, db)
        outs.append((pre.cpu(), dw.cpu(), db.cpu(), dx[:, :4096].cpu()))
        if D > 4096:
            assert not dx[:, 4096:].any()
    for a, c in zip(*outs):
        assert torch.equal(a, c)


def test_bf16_tiles_give_the_bits_of_fp32_tiles():
    """bf16 X at 4096 < D <= 8192 runs the forward and dW over 4-token tiles of raw bf16 values
    (each widened exactly before use); the same values given as fp32 X run two-token fp32 tiles.
    pre, dW, db and dX are bit-identical (same values, same order of every sum), and pre matches
    the oracle; ragged B."""
    L, idx, w, b, x, dy = make_case(8192, 12000, 12, 8, 45, x_dtype=torch.bfloat16, seed=13)
    rt = _rt(L, idx, LevelSpec("mean", activation="relu"))
    wd, bd = w.to(DEV), b.to(DEV)
    outs = []
    for xd in (x.to(DEV), x.float().to(DEV)):
        pre = rt.forward(xd, wd, bd)["pre"]
        dw = torch.zeros(L.weight_shape, device=DEV)
        db = torch.zeros(L.bias_shape, device=DEV)
        dx = rt.backward(xd, wd, bd, dy.to(DEV), {}, "minimal_stats", dw, db)
        outs.append((pre.cpu(), dw.cpu(), db.cpu(), dx.float().cpu()))
    for a, c in zip(*outs):
        assert torch.equal(a, c)
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    want, mag = O.forward(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group, "relu", "mean", with_mag=True)
    assert_parity(outs[0][0].numpy(), want, mag, what="pre")
