"""Parity at the BASELINE configurations' full sizes (one MI355X), through the drop-in layer and
the C ABI, against the float64 CPU oracle on identical seeded inputs.

* C1 (B 64, D 1024, N 1,048,576, pools of 256) is checked whole: three training steps of
  SparsePoolingLayer + FusedAdamW, every step's forward, dX, dW and db against the oracle and every
  AdamW update against the oracle's update of the same gradient and moments.
* C2..C5 run at their full N (100,663,296 neurons at fan-in 8; 50,331,648 at fan-in 16), where
  weight and mask byte offsets pass 2^31: the forward of the whole layer is compared on 24 pools
  (the first, the last three and 20 seeded ones) and the backward with dY non-zero only on those
  pools, whose dX the oracle computes from those pools alone.

fp32 bar: conftest.assert_parity (elementwise 1e-6 + 1e-5 * sum|terms|, plus the whole-tensor
relative error <= 1e-5); AdamW: rel 1e-5 / abs 1e-6 elementwise against the oracle's fp32 step.
"""
import numpy as np
import pytest
import torch

from conftest import assert_close, assert_parity, gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

from granulelayer_amd import FusedAdamW, LevelSpec, PhysicalPlan, SparsePoolingLayer  # noqa: E402
from granulelayer_amd.autograd import Level1Runtime  # noqa: E402
from granulelayer_amd.synthetic import CONFIGS, make_problem  # noqa: E402
from oracle import oracle as O  # noqa: E402

DEV = "cuda"
LR, BETAS, EPS = 1e-3, (0.9, 0.999), 1e-8


def _flat(idx, w, b, K):
    return (idx.reshape(-1, K).cpu().numpy(), w.detach().reshape(-1, K).cpu().numpy(),
            b.detach().reshape(-1).cpu().numpy())


def test_c1_full_layer_three_train_steps_match_oracle():
    """BASELINE configs[0] whole on the GPU: SparsePoolingLayer(1024, 1,048,576, 4096, fan-in 8,
    sum of relu) with main_grad and FusedAdamW(fp32 moments, lr 1e-3, betas 0.9/0.999, eps 1e-8),
    three steps.  Each step: y, dX (x.grad), dW and db (main_grad) against the oracle of the current
    parameters; then the AdamW step against the oracle's fp32 step of the same gradient."""
    pr = make_problem("C1", device="cpu", seed=0)
    L = pr.layout
    K, S = L.fan_in, L.slots_per_group
    assert (pr.B, L.input_dim, L.hidden_dim, L.groups, S) == (64, 1024, 1_048_576, 4096, 256)
    lay = SparsePoolingLayer(L.input_dim, L.hidden_dim, L.groups, fan_in=K, shared_neurons=None, pooling="sum",
                             dtype=torch.float32, device=DEV, seed=0)
    with torch.no_grad():
        lay.indices.copy_(pr.idx.to(DEV))
        lay.weight.copy_(pr.w.to(DEV))
        lay.bias.copy_(pr.b.to(DEV))
    lay.enable_main_grad()
    opt = FusedAdamW(lay.parameters(), lr=LR, betas=BETAS, eps=EPS, weight_decay=0.0, moments="fp32")
    counts = L.counts_tensor("cpu").numpy()
    xn, dyn = pr.x.numpy(), pr.dy.numpy()
    m = {p: np.zeros(p.numel(), np.float32) for p in (lay.weight, lay.bias)}
    v = {p: np.zeros(p.numel(), np.float32) for p in (lay.weight, lay.bias)}
    for t in range(1, 4):
        fi, fw, fb = _flat(lay.indices, lay.weight, lay.bias, K)
        x = pr.x.to(DEV).requires_grad_(True)
        y = lay(x)
        y.backward(pr.dy.to(DEV))
        want, mag = O.forward(xn, fi, fw, fb, counts, S, "relu", "sum", with_mag=True)
        assert_parity(y.detach().cpu().numpy(), want, mag, what=f"step {t} y")
        wdW, wdb, wdX, bnd = O.backward(xn, fi, fw, fb, counts, S, dyn, "relu", "sum", with_bounds=True)
        (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
        assert_parity(x.grad.cpu().numpy(), wdX, mX, uX, what=f"step {t} dX")
        assert_parity(lay.weight.main_grad.cpu().numpy().reshape(-1, K), wdW, mW, uW, what=f"step {t} dW")
        assert_parity(lay.bias.main_grad.cpu().numpy().reshape(-1), wdb, mb, ub, what=f"step {t} db")
        # the oracle's AdamW step on the same parameters, gradient and moments
        want_p = {}
        for p in (lay.weight, lay.bias):
            po = p.detach().cpu().numpy().reshape(-1).copy()
            O.adam(po, p.main_grad.cpu().numpy().reshape(-1).copy(), m[p], v[p], LR, BETAS[0], BETAS[1], EPS, 0.0, t)
            want_p[p] = po
        opt.step()
        for name, p in (("W", lay.weight), ("b", lay.bias)):
            st = opt.state[p]
            assert_close(p.detach().cpu().numpy().reshape(-1), want_p[p], what=f"step {t} AdamW {name}")
            assert_close(st["m"].cpu().numpy().reshape(-1), m[p], what=f"step {t} m {name}")
            assert_close(st["v"].cpu().numpy().reshape(-1), v[p], what=f"step {t} v {name}")
            assert float(p.main_grad.abs().max()) == 0.0, "fused zero_grad"
            same = float((p.detach().cpu().numpy().reshape(-1) == want_p[p]).mean())
            print(f"C1 step {t} {name}: {same * 100:.4f}% of parameters bitwise equal to the oracle")


def _pools(G, n=24, seed=0):
    rng = np.random.default_rng(seed)
    extra = np.setdiff1d(rng.choice(G, 2 * n, replace=False), [0, G - 3, G - 2, G - 1])[:n - 4]
    return np.sort(np.concatenate([[0, G - 3, G - 2, G - 1], extra]))


@pytest.mark.parametrize("cfg", ["C2", "C3", "C4", "C5"])
def test_full_size_layer_on_sampled_pools(cfg):
    """The whole BASELINE layer on the GPU (N = 100,663,296 neurons at fan-in 8, 50,331,648 at fan-in
    16, so byte offsets of W, dW and the activation masks pass 2^31): forward pre of 24 pools (the
    first, the last three, 20 seeded) against the oracle run on those pools; backward with dY zero
    outside them, dW / db of those pools and the full dX against the oracle's backward of those
    pools, and zero dW on pools with zero dY."""
    c = CONFIGS[cfg]
    pr = make_problem(cfg, device=DEV, seed=0)
    L = pr.layout
    K, S, G = L.fan_in, L.slots_per_group, L.groups
    assert L.hidden_dim == c["N"] and G * S * K * 4 > 2**31
    rt = Level1Runtime(L, pr.idx, LevelSpec("sum"), PhysicalPlan())
    pre = rt.forward(pr.x, pr.w, pr.b)["pre"]
    pools = _pools(G)
    dy = torch.zeros_like(pr.dy)
    sel = torch.from_numpy(pools).to(DEV)
    dy[:, sel] = pr.dy[:, sel]
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(pr.x, pr.w, pr.b, dy, {}, "minimal_stats", dw, db).cpu().numpy()
    slots = torch.cat([torch.arange(g * S, (g + 1) * S, device=DEV) for g in pools.tolist()])
    fi = pr.idx.reshape(-1, K)[slots].cpu().numpy()
    fw = pr.w.reshape(-1, K)[slots].cpu().numpy()
    fb = pr.b.reshape(-1)[slots].cpu().numpy()
    counts = np.full(len(pools), S, np.int32)
    xn = pr.x.float().cpu().numpy()  # bf16 inputs widened exactly, as the kernels do
    want, mag = O.forward(xn, fi, fw, fb, counts, S, "relu", "sum", with_mag=True)
    assert_parity(pre[:, sel].cpu().numpy(), want, mag, what=f"{cfg} pre (full layer, sampled pools)")
    wdW, wdb, wdX, bnd = O.backward(xn, fi, fw, fb, counts, S, pr.dy[:, sel].cpu().numpy(), "relu", "sum",
                                    with_bounds=True)
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_parity(dw.reshape(-1, K)[slots].cpu().numpy(), wdW, mW, uW, what=f"{cfg} dW (sampled pools)")
    assert_parity(db.reshape(-1)[slots].cpu().numpy(), wdb, mb, ub, what=f"{cfg} db (sampled pools)")
    assert_parity(dx, wdX, mX, uX, what=f"{cfg} dX (dY on sampled pools)")
    others = torch.from_numpy(np.setdiff1d(np.arange(G - 200, G), pools)).to(DEV)
    assert float(dw.reshape(G, -1)[others].abs().max()) == 0.0, "pools with zero dY get zero dW"
    assert float(db.reshape(G, -1)[others].abs().max()) == 0.0


@pytest.mark.parametrize("pool,k", [("sum", 0), ("max", 1), ("topk_mean", 8)])
def test_forward_token_chunks_are_bit_identical(pool, k):
    """A small part budget makes the forward run several token passes (each reloading the chunk
    parameters); pre and the selected slots are bit-identical to the one-pass forward."""
    from test_gpu_parity import make_case

    D, H, G, K, B = 512, 40000, 40, 8, 203
    L, idx, w, b, x, _ = make_case(D, H, G, K, B)
    spec = LevelSpec(pool, activation="relu", k=k) if pool == "topk_mean" else LevelSpec(pool, activation="relu")
    outs = []
    for budget in (None, 8 * 2**10):
        kw = {} if budget is None else {"workspace_budget": budget}
        rt = Level1Runtime(L, idx.to(DEV), spec, PhysicalPlan(), **kw)
        outs.append((rt.forward(x.to(DEV), w.to(DEV), b.to(DEV), track_ids=pool != "sum"),
                     rt.last_info["workspace_bytes"]))
    (one, ws1), (many, ws2) = outs
    assert ws2 < ws1 / 4, "the small budget must split the batch into several passes"
    assert one.keys() == many.keys()
    for key in one:
        assert torch.equal(one[key], many[key]), f"{key} differs between one and several token passes"


# pools of 1024 (4 per forward workgroup at 16 waves, 3 at 12, 2 at 8) and of 300 inside windows
WIN_SEL_CASES = [(2048, 8192, 8, 8, 37, 256), (1536, 4800, 16, 8, 70, 120)]


@pytest.mark.parametrize("case", WIN_SEL_CASES, ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}w{c[5]}")
@pytest.mark.parametrize("pool,k", [("max", 1), ("topk_mean", 8), ("topk_mean", 64)])
def test_window_staging_of_selection_pools(case, pool, k):
    """The window-staged forward with the max and top-k tiles (12 and 8 waves per workgroup, so a
    different number of pools per workgroup than sum): pre and the selected slots bit-identical to
    full staging, the window kernel in the trace, and the slots equal to the oracle's wherever the
    selection's lead exceeds fp32 rounding."""
    from granulelayer_amd import _native as N
    from granulelayer_amd.backend import HipBackend
    from test_gpu_parity import flat, make_window_case

    D, H, G, K, B, width = case
    L, idx, w, b, x, _ = make_window_case(D, H, G, K, B, width)
    spec = LevelSpec(pool, activation="identity", k=k) if pool == "topk_mean" else LevelSpec(pool, activation="identity")
    key = "winner" if pool == "max" else "topk_slot"
    be = HipBackend.get()
    outs = {}
    try:
        for ws in (True, False):
            be.window_staging = ws
            rt = Level1Runtime(L, idx.to(DEV), spec, PhysicalPlan())
            with N.KernelTrace() as tr:
                out = rt.forward(x.to(DEV), w.to(DEV), b.to(DEV), track_ids=True)
            names = set(tr.times_ms())
            assert ("fwd_kernel_win" if ws else "fwd_kernel") in names, f"window_staging={ws}: ran {sorted(names)}"
            outs[ws] = {kk: t.cpu() for kk, t in out.items()}
    finally:
        be.window_staging = True
    for kk in outs[True]:
        assert torch.equal(outs[True][kk], outs[False][kk]), f"{kk} differs between window and full staging"
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    xn = x.float().numpy()
    if pool == "max":
        want, wsl, gap = O.forward_max(xn, fi, fw, fb, counts, L.slots_per_group, "identity")
        got = outs[True][key].numpy()
    else:
        want, wsl, gap = O.forward_topk(xn, fi, fw, fb, counts, L.slots_per_group, k, "identity")
        got, wsl = np.sort(outs[True][key].numpy(), -1), np.sort(wsl, -1)
    assert_close(outs[True]["pre"].numpy(), want, rtol=1e-5, atol=1e-6, what=f"{pool} pre")
    clear = gap > 2e-6
    assert clear.mean() > 0.95
    assert (got[clear] == wsl[clear]).all(), f"{int((got[clear] != wsl[clear]).sum())} selected slots differ"


@pytest.mark.parametrize("pooling", ["max", {"type": "topk_mean", "k": 8}], ids=["max", "topk8"])
def test_selection_backward_over_the_checkpoint_budget(pooling, monkeypatch):
    """When the batch's selection ids exceed the checkpoint budget, save_winners falls back to
    minimal_stats (last_info['policy_fallback']) and the backward recomputes the ids one token chunk
    at a time (autograd.py:45-56, 255-259, 329-343); the gradients equal the oracle's backward of the
    layer's own selection.  The budgets are shrunk so a small layer exercises the path."""
    import granulelayer_amd.autograd as A
    from test_gpu_parity import flat

    D, H, G, K, B = 256, 12000, 12, 8, 100
    topk = pooling != "max"
    kk = 8 if topk else 1
    monkeypatch.setattr(A, "CHECKPOINT_BUDGET", 40 * G * kk * 4)
    monkeypatch.setattr(A, "RECOMPUTE_CHUNK_BYTES", 32 * G * kk * 4)
    lay = SparsePoolingLayer(D, H, G, fan_in=K, shared_neurons=None, pooling=pooling, checkpoint_policy="save_winners",
                             dtype=torch.float32, device=DEV, seed=8, bias_std=0.2)
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(B, D, generator=gen).to(DEV).requires_grad_(True)
    dy = torch.randn(B, G, generator=gen).to(DEV)
    y = lay(x)
    assert "policy_fallback" in lay.last_info
    (y * dy).sum().backward()
    info = lay.last_info
    assert info["backward_token_chunks"] == -(-B // A.recompute_chunk(lay._rt)) > 1
    L = lay.layout
    fi, fw, fb = flat(L, lay.indices.cpu(), lay.weight.detach().cpu(), lay.bias.detach().cpu())
    counts = L.counts_tensor("cpu").numpy()
    xn = x.detach().cpu().numpy()
    # the layer's own selection (recomputed, as the chunked backward did), so a near-tie between
    # neurons never decides the comparison
    st = lay._rt.forward(x.detach(), lay.weight.detach(), lay.bias.detach(), track_ids=True)
    slots = st["topk_slot" if topk else "winner"].cpu().numpy()
    if topk:
        want, _, _ = O.forward_topk(xn, fi, fw, fb, counts, L.slots_per_group, 8)
        g_pre = dy.cpu().numpy()
    else:
        want, _, _ = O.forward_max(xn, fi, fw, fb, counts, L.slots_per_group, "identity")
        g_pre = (dy.cpu().numpy() * (st["pre"].cpu().numpy() > 0)).astype(np.float32)  # relu out-activation
        want = np.maximum(want, 0.0)
    assert_close(y.detach().cpu().numpy(), want, rtol=1e-5, atol=1e-6, what="y")
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_events(xn, fi, fw, fb, counts, L.slots_per_group, g_pre,
                                                    slots, "identity", topk=topk)
    assert_parity(x.grad.cpu().numpy(), wdX, mX, what="dx")
    assert_parity(lay.weight.grad.cpu().numpy().reshape(-1, K), wdW, mW, what="dW")
    assert_parity(lay.bias.grad.cpu().numpy().reshape(-1), wdb, mb, what="db")


def test_adam_at_the_c4_size_matches_the_oracle_on_a_sample():
    """gl_adam over C4's 805,306,368-element weight stream (3.2 GB per array, byte offsets past
    2^31): two steps, then a seeded sample of elements -- the first and last 4096, 4096 around
    element 2^29 (byte 2^31), 65,536 random -- against oracle.adam on the same elements (the update
    is elementwise, so a sample evolves on its own).  Every sampled index is checked to lie in
    [0, n) on the host before it reaches the device."""
    from granulelayer_amd.backend import HipBackend
    from oracle import oracle as O

    n = 805_306_368
    gen = torch.Generator(device=DEV).manual_seed(21)
    p = torch.randn(n, generator=gen, device=DEV)
    m = torch.randn(n, generator=gen, device=DEV) * 0.01
    v = torch.rand(n, generator=gen, device=DEV) * 1e-4
    rng = np.random.default_rng(5)
    parts = [np.arange(4096), np.arange(n - 4096, n), np.arange((1 << 29) - 2048, (1 << 29) + 2048),
             rng.integers(0, n, 65536)]
    idx = np.unique(np.concatenate(parts))
    assert idx.min() >= 0 and idx.max() < n
    sample = torch.as_tensor(idx, device=DEV)
    po, mo, vo = (t[sample].cpu().numpy().copy() for t in (p, m, v))
    be = HipBackend.get()
    for t in (1, 2):
        g = torch.randn(n, generator=gen, device=DEV)
        go = g[sample].cpu().numpy().copy()
        be.adam(p, g, m, v, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1 - 0.9 ** t, 1 - 0.999 ** t)
        O.adam(po, go, mo, vo, 1e-3, 0.9, 0.999, 1e-8, 0.01, t)
        assert float(g[sample].abs().max()) == 0.0 and float(g[-4096:].abs().max()) == 0.0, "fused zero_grad"
        del g
    for name, got, want in (("p", p, po), ("m", m, mo), ("v", v, vo)):
        gs = got[sample].cpu().numpy()
        assert_close(gs, want, what=f"adam {name} (C4 size, sampled)")
        print(f"adam C4 size {name}: {(gs == want).mean() * 100:.3f}% of the sample bitwise equal to the oracle")
