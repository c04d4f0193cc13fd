"""The forward's ReLU bits handed to the backward (GlFwdArgs / GlBwdArgs.relu_mask,
PhysicalPlan(relu_bits="keep")).

The reference's backward recomputes z to find the ReLU mask (sparse_pooling/kernels/
triton_fused.py:364-374).  With relu_bits="keep" the forward also stores the bit z > 0 of every
(token, neuron) and the dW pass reads it instead of recomputing z.  The decision is the same
fp32 compare of the same z (same operands, same summation order), so:

* through Level1Runtime, dW, db and dX from the kept bits equal those of the recompute bit for bit,
  across every tile format that has bits (fp32 tiles, bf16 tiles, pool windows, X gathered from
  global memory), several forward token passes, two backward token chunks and ragged batches; the
  layers without bits (two-token fp32 tiles, fan-in 16, GELU) report a size of 0;
* through the layer, a relu_bits="keep" training step matches the float64 oracle and keeps the
  bits in its checkpoint, and the default plan keeps none (the reference's O(B x G) checkpoint).
"""
import numpy as np
import pytest
import torch

from conftest import assert_parity, gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

from granulelayer_amd import LevelSpec, PhysicalPlan, SparsePoolingLayer  # noqa: E402
from granulelayer_amd._native import KernelTrace  # noqa: E402
from granulelayer_amd.autograd import Level1Runtime  # noqa: E402
from oracle import oracle as O  # noqa: E402

DEV = "cuda"

# D, H, G, B, x dtype, window width (0: uniform indices), workspace budget (0: default)
CASES = [
    (1024, 65536, 64, 301, torch.float32, 0, 0),        # fp32 tiles, two workgroups per CU; ragged B
    (1024, 65536, 64, 300, torch.float32, 0, 1 << 16),  # five forward token passes of 64
    (512, 20000, 20, 1100, torch.float32, 0, 0),        # two backward token chunks
    (6000, 30000, 30, 70, torch.bfloat16, 0, 0),        # bf16 tiles (D > 4096)
    (2048, 8192, 8, 64, torch.bfloat16, 256, 0),        # bf16 pool windows
    (2048, 8192, 8, 37, torch.float32, 256, 0),         # fp32 pool windows
    (12000, 8192, 8, 9, torch.float32, 0, 0),           # X gathered from global memory
]


def _case(D, H, G, B, xdt, width, seed=0):
    from test_gpu_parity import make_case, make_window_case

    if width:
        return make_window_case(D, H, G, 8, B, width, seed=seed, x_dtype=xdt)
    return make_case(D, H, G, 8, B, seed=seed, x_dtype=xdt)


@pytest.mark.parametrize("pool", ["sum", "mean"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}B{c[3]}{str(c[4])[6:]}w{c[5]}b{c[6]}")
def test_relu_bits_give_the_bits_of_the_recompute(case, pool):
    D, H, G, B, xdt, width, budget = case
    L, idx, w, b, x, dy = _case(D, H, G, B, xdt, width)
    rt = Level1Runtime(L, idx.to(DEV), LevelSpec(pool, activation="relu"), PhysicalPlan(),
                       workspace_budget=budget or None)
    xd, wd, bd, dyd = x.to(DEV), w.to(DEV), b.to(DEV), dy.to(DEV)
    res = {}
    for keep in (True, False):
        dw = torch.zeros(L.weight_shape, device=DEV)
        db = torch.zeros(L.bias_shape, device=DEV)
        out = rt.forward(xd, wd, bd, relu_mask=keep)
        assert ("relu_mask" in out) == keep
        if keep:
            assert out["relu_mask"].numel() == G * -(-L.slots_per_group // 256) * -(-B // 4) * 128
        with KernelTrace() as tr:
            dx = rt.backward(xd, wd, bd, dyd, out, "minimal_stats", dw, db)
        torch.cuda.synchronize()
        assert rt.last_info["backward_relu_mask"] == keep
        assert any(n.startswith("bwd_w_kernel") for n in tr.times_ms())
        res[keep] = [t.cpu() for t in (out["pre"], dw, db, dx)]
    for name, a, c in zip(("pre", "dW", "db", "dX"), res[True], res[False]):
        assert torch.equal(a, c), f"{name}: kept ReLU bits differ from the recompute"


@pytest.mark.parametrize("D,K,act,xdt", [(6000, 8, "relu", torch.float32), (256, 16, "relu", torch.float32),
                                         (256, 8, "gelu", torch.float32), (256, 8, "identity", torch.float32)])
def test_layers_without_relu_bits_keep_none(D, K, act, xdt):
    """Two-token fp32 tiles (4096 < D <= 8192), fan-in 16 and non-ReLU neurons have no bits: the
    forward returns none and the backward recomputes."""
    from test_gpu_parity import make_case

    L, idx, w, b, x, dy = make_case(D, 4096, 8, K, 20, x_dtype=xdt)
    rt = Level1Runtime(L, idx.to(DEV), LevelSpec("sum", activation=act), PhysicalPlan())
    out = rt.forward(x.to(DEV), w.to(DEV), b.to(DEV), relu_mask=True)
    assert "relu_mask" not in out


@pytest.mark.parametrize("pool", ["sum", "mean"])
def test_layer_with_relu_bits_matches_oracle(pool):
    """SparsePoolingLayer(plan=PhysicalPlan(relu_bits="keep")): forward, dX, dW (main_grad) and db
    against the float64 oracle; the checkpoint holds the bits; the default plan keeps none."""
    D, H, G, B = 1024, 65536, 64, 130
    lay = SparsePoolingLayer(D, H, G, shared_neurons=None, pooling=pool, dtype=torch.float32, device=DEV, seed=3,
                             bias_std=0.3, plan=PhysicalPlan(relu_bits="keep"))
    lay.enable_main_grad()
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(B, D, generator=gen).to(DEV).requires_grad_(True)
    dy = torch.randn(B, G, generator=gen).to(DEV)
    y = lay(x)
    info = lay.last_info
    y.backward(dy)
    assert lay.last_info["backward_relu_mask"]
    L = lay.layout
    bits = G * (L.slots_per_group // 256) * (-(-B // 4)) * 128
    assert info["checkpoint_bytes"] == B * G * 4 + bits
    K = L.fan_in
    idx = lay.indices.cpu().reshape(-1, K).numpy()
    w = lay.weight.detach().cpu().reshape(-1, K).numpy()
    b = lay.bias.detach().cpu().reshape(-1).numpy()
    counts = L.counts_tensor("cpu").numpy()
    xn = x.detach().cpu().numpy()
    want, mag = O.forward(xn, idx, w, b, counts, L.slots_per_group, "relu", pool, with_mag=True)
    assert_parity(y.detach().cpu().numpy(), want, mag, what="y")
    wdW, wdb, wdX, bnd = O.backward(xn, idx, w, b, counts, L.slots_per_group, dy.cpu().numpy(), "relu", pool,
                                    with_bounds=True)
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_parity(x.grad.cpu().numpy(), wdX, mX, uX, what="dX")
    assert_parity(lay.weight.main_grad.cpu().numpy().reshape(-1, K), wdW, mW, uW, what="dW")
    assert_parity(lay.bias.main_grad.cpu().numpy().reshape(-1), wdb, mb, ub, what="db")

    with torch.no_grad():  # no backward can follow: no bits
        lay(x)
    assert not lay.last_info["forward_relu_mask"]

    dflt = SparsePoolingLayer(D, H, G, shared_neurons=None, pooling=pool, dtype=torch.float32, device=DEV, seed=3)
    dflt.enable_main_grad()
    dflt(x).sum().backward()
    assert dflt.last_info["checkpoint_bytes"] == B * G * 4
    assert not dflt.last_info["backward_relu_mask"]
