"""LogMeanExp, power mean and softmax-weighted pooling on the GPU (pytorch_reference.py:80-100;
backward kernels/ops.py:242-262, triton_fused.py:364-399) against the float64 oracle on identical
seeded inputs: forward pre and the log-normaliser L2, backward dX / dW / db, the layer's autograd
under its checkpoint policies, bitwise determinism, two backward token chunks and D > 4096, the
power mean at every integer p the kernels take as a literal, and the dz budget's token chunks.

fp32 bar: conftest.assert_parity with the oracle's error scales (elementwise 1e-6 + 1e-5 * mag and
a whole-tensor relative error <= 1e-5)."""
import numpy as np
import pytest
import torch

from conftest import assert_parity, gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

from granulelayer_amd import LevelSpec, PhysicalPlan, SparsePoolingLayer  # noqa: E402
from granulelayer_amd.autograd import Level1Runtime  # noqa: E402
from oracle import oracle as O  # noqa: E402

DEV = "cuda"

OPS = [("logmeanexp", 1.0, "identity"), ("logmeanexp", 0.5, "relu"), ("power_mean", 2.0, "relu"),
       ("power_mean", 3.0, "relu"), ("softmax_weighted", 1.0, "identity"), ("softmax_weighted", 2.0, "relu"),
       ("logmeanexp", 0.7, "gelu"), ("softmax_weighted", 1.5, "gelu")]
CASES = [
    # D, H, G, K, B, x dtype
    (64, 3000, 8, 8, 37, torch.float32),
    (1024, 20011, 16, 8, 64, torch.bfloat16),
    (96, 5000, 7, 16, 33, torch.float32),
    (1024, 65536, 64, 8, 130, torch.float32),  # one 130-token chunk: the dense dX at 4 tokens per lane
]


def _spec(pool, param, act):
    kw = {"logmeanexp": "temperature", "power_mean": "p", "softmax_weighted": "beta"}[pool]
    return LevelSpec(pool, activation=act, **{kw: param})


def _case(case, seed=0):
    from test_gpu_parity import make_case

    D, H, G, K, B, xdt = case
    return make_case(D, H, G, K, B, seed=seed, x_dtype=xdt, bias_std=0.3)


def _flat(L, idx, w, b):
    K = L.fan_in
    return idx.reshape(-1, K).numpy(), w.reshape(-1, K).numpy(), b.reshape(-1).numpy()


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}{str(c[5])[6:]}")
@pytest.mark.parametrize("pool,param,act", OPS, ids=lambda v: str(v))
def test_smooth_forward_and_backward_match_oracle(case, pool, param, act):
    L, idx, w, b, x, dy = _case(case)
    rt = Level1Runtime(L, idx.to(DEV), _spec(pool, param, act), PhysicalPlan())
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    out = rt.forward(xd, wd, bd)
    fi, fw, fb = _flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    xn = x.float().numpy()
    want, lse, mag = O.forward_smooth(xn, fi, fw, fb, counts, L.slots_per_group, pool, param, act)
    assert_parity(out["pre"].cpu().numpy(), want, mag, what=f"{pool} pre")
    if pool != "power_mean":
        assert_parity(out["L2"].cpu().numpy(), lse, np.abs(lse) + mag, what=f"{pool} L2")
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(xd, wd, bd, dy.to(DEV), out, "minimal_stats", dw, db).cpu().numpy()
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_smooth(xn, fi, fw, fb, counts, L.slots_per_group, dy.numpy(), pool,
                                                    param, act)
    K = L.fan_in
    assert_parity(dx, wdX, mX, what=f"{pool} dX")
    assert_parity(dw.cpu().numpy().reshape(-1, K), wdW, mW, what=f"{pool} dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, what=f"{pool} db")
    # deterministic: a second backward gives the same bits
    dw2, db2 = torch.zeros_like(dw), torch.zeros_like(db)
    dx2 = rt.backward(xd, wd, bd, dy.to(DEV), out, "minimal_stats", dw2, db2).cpu().numpy()
    assert np.array_equal(dx, dx2) and torch.equal(dw, dw2) and torch.equal(db, db2)


@pytest.mark.parametrize("pool,param,act", [OPS[0], OPS[2], OPS[4]], ids=lambda v: str(v))
@pytest.mark.parametrize("policy", ["minimal_stats", "recompute_stats"])
def test_smooth_layer_autograd_policies(pool, param, act, policy):
    """SparsePoolingLayer with a smooth operator: minimal_stats keeps pre (and L2 for softmax-weighted,
    autograd.py:366-377), recompute_stats reruns the forward in backward; both give the oracle's
    gradients."""
    D, H, G, K, B = 256, 12000, 12, 8, 40
    pooling = {"type": pool, {"logmeanexp": "temperature", "power_mean": "p", "softmax_weighted": "beta"}[pool]: param,
               "activation": act}
    lay = SparsePoolingLayer(D, H, G, fan_in=K, shared_neurons=None, pooling=pooling, checkpoint_policy=policy,
                             dtype=torch.float32, device=DEV, seed=6, bias_std=0.2)
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(B, D, generator=gen).to(DEV).requires_grad_(True)
    dy = torch.randn(B, G, generator=gen).to(DEV)
    y = lay(x)
    (y * dy).sum().backward()
    L = lay.layout
    fi, fw, fb = _flat(L, lay.indices.cpu(), lay.weight.detach().cpu(), lay.bias.detach().cpu())
    counts = L.counts_tensor("cpu").numpy()
    xn = x.detach().cpu().numpy()
    want, _, mag = O.forward_smooth(xn, fi, fw, fb, counts, L.slots_per_group, pool, param, act)
    assert_parity(y.detach().cpu().numpy(), want, mag, what="y")
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_smooth(xn, fi, fw, fb, counts, L.slots_per_group, dy.cpu().numpy(), pool,
                                                    param, act)
    assert_parity(x.grad.cpu().numpy(), wdX, mX, what="dx")
    assert_parity(lay.weight.grad.cpu().numpy().reshape(-1, K), wdW, mW, what="dW")
    assert_parity(lay.bias.grad.cpu().numpy().reshape(-1), wdb, mb, what="db")
    assert lay.last_info["recomputed_stats"] == (policy == "recompute_stats")


@pytest.mark.parametrize("case", [(2048, 8000, 8, 8, 1100, torch.float32), (6000, 9000, 9, 8, 20, torch.bfloat16)],
                         ids=["two-token-chunks", "D6000"])
@pytest.mark.parametrize("pool,param,act", [OPS[1], OPS[3], OPS[5]], ids=lambda v: str(v))
def test_smooth_backward_chunks_and_wide_inputs(case, pool, param, act):
    """B = 1100 (two backward token chunks: the coefficients and dz of the second start at b0 = 1024)
    and D = 6000 (single-buffered token tiles)."""
    L, idx, w, b, x, dy = _case(case, seed=3)
    rt = Level1Runtime(L, idx.to(DEV), _spec(pool, param, act), PhysicalPlan())
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    out = rt.forward(xd, wd, bd)
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(xd, wd, bd, dy.to(DEV), out, "minimal_stats", dw, db).cpu().numpy()
    fi, fw, fb = _flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    xn = x.float().numpy()
    want, _, mag = O.forward_smooth(xn, fi, fw, fb, counts, L.slots_per_group, pool, param, act)
    assert_parity(out["pre"].cpu().numpy(), want, mag, what="pre")
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_smooth(xn, fi, fw, fb, counts, L.slots_per_group, dy.numpy(), pool,
                                                    param, act)
    assert_parity(dx, wdX, mX, what="dX")
    assert_parity(dw.cpu().numpy().reshape(-1, L.fan_in), wdW, mW, what="dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, what="db")


@pytest.mark.parametrize("pool,param,act", [OPS[0], OPS[3], OPS[4]], ids=lambda v: str(v))
def test_smooth_backward_dz_budget_sets_the_token_chunks(pool, param, act):
    """The dz budget only chunks the tokens: a budget below one 64-token chunk runs B = 200 as four
    chunks (64, 64, 64, 8) with a smaller workspace, and both runs give the oracle's gradients;
    dX of a token never crosses a chunk."""
    L, idx, w, b, x, dy = _case((512, 6000, 6, 8, 200, torch.float32), seed=5)
    xd, wd, bd, dyd = x.to(DEV), w.to(DEV), b.to(DEV), dy.to(DEV)
    fi, fw, fb = _flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_smooth(x.numpy(), fi, fw, fb, counts, L.slots_per_group, dy.numpy(), pool,
                                                    param, act)
    info = []
    for budget in (1, 2**30):
        rt = Level1Runtime(L, idx.to(DEV), _spec(pool, param, act), PhysicalPlan(), workspace_budget=budget)
        out = rt.forward(xd, wd, bd)
        dw = torch.zeros(L.weight_shape, device=DEV)
        db = torch.zeros(L.bias_shape, device=DEV)
        dx = rt.backward(xd, wd, bd, dyd, out, "minimal_stats", dw, db).cpu().numpy()
        assert_parity(dx, wdX, mX, what=f"dX at budget {budget}")
        assert_parity(dw.cpu().numpy().reshape(-1, L.fan_in), wdW, mW, what=f"dW at budget {budget}")
        assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, what=f"db at budget {budget}")
        info.append(rt.last_info["backward_workspace_bytes"])
    # one 64-token chunk of dz against the whole B = 200 (cap 256) at once
    assert info[0] < info[1]
    assert info[1] - info[0] >= L.groups * L.slots_per_group * (256 - 64) * 4


@pytest.mark.parametrize("B,passes", [(128, 2), (200, 4)])
@pytest.mark.parametrize("pool,param,act", [OPS[1], OPS[3], OPS[4]], ids=lambda v: str(v))
def test_smooth_dense_dx_in_unit_range_passes(B, passes, pool, param, act):
    """A layer large enough for the dense dX's short unit ranges (2.1 M edges into 64 inputs, 1024
    pools): the ranges run as 2 passes at 2 tokens per lane (B = 128) and 4 at 4 (B = 200), each
    pass's partials reduced onto the previous passes' dX; gradients against the oracle, and a second
    backward bit-identical."""
    from granulelayer_amd._native import KernelTrace

    L, idx, w, b, x, dy = _case((64, 262144, 1024, 8, B, torch.float32), seed=11)
    rt = Level1Runtime(L, idx.to(DEV), _spec(pool, param, act), PhysicalPlan())
    xd, wd, bd, dyd = x.to(DEV), w.to(DEV), b.to(DEV), dy.to(DEV)
    out = rt.forward(xd, wd, bd)
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    with KernelTrace(max_launches=256) as tr:
        dx = rt.backward(xd, wd, bd, dyd, out, "minimal_stats", dw, db)
        torch.cuda.synchronize()
    launches = {k: len(v) for k, v in tr.times_ms().items()}
    assert launches.get("dx_dense_kernel") == passes and launches.get("dx_reduce_kernel") == passes, launches
    dx = dx.cpu().numpy()
    fi, fw, fb = _flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_smooth(x.numpy(), fi, fw, fb, counts, L.slots_per_group, dy.numpy(), pool,
                                                    param, act)
    assert_parity(dx, wdX, mX, what="dX")
    assert_parity(dw.cpu().numpy().reshape(-1, L.fan_in), wdW, mW, what="dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, what="db")
    dw2, db2 = torch.zeros_like(dw), torch.zeros_like(db)
    dx2 = rt.backward(xd, wd, bd, dyd, out, "minimal_stats", dw2, db2).cpu().numpy()
    assert np.array_equal(dx, dx2) and torch.equal(dw, dw2) and torch.equal(db, db2)



@pytest.mark.parametrize("case", [CASES[0], CASES[2]], ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}")
@pytest.mark.parametrize("p", [1.0, 4.0, 8.0])
def test_power_mean_integer_p(case, p):
    """The power mean's integer p (1, 4, 8; 2 in the main test) runs kernels where p is a literal:
    forward pre and backward dX / dW / db against the oracle."""
    L, idx, w, b, x, dy = _case(case, seed=9)
    rt = Level1Runtime(L, idx.to(DEV), _spec("power_mean", p, "relu"), PhysicalPlan())
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    out = rt.forward(xd, wd, bd)
    fi, fw, fb = _flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    xn = x.float().numpy()
    want, _, mag = O.forward_smooth(xn, fi, fw, fb, counts, L.slots_per_group, "power_mean", p, "relu")
    assert_parity(out["pre"].cpu().numpy(), want, mag, what=f"p {p} pre")
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(xd, wd, bd, dy.to(DEV), out, "minimal_stats", dw, db).cpu().numpy()
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_smooth(xn, fi, fw, fb, counts, L.slots_per_group, dy.numpy(),
                                                    "power_mean", p, "relu")
    assert_parity(dx, wdX, mX, what=f"p {p} dX")
    assert_parity(dw.cpu().numpy().reshape(-1, L.fan_in), wdW, mW, what=f"p {p} dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, what=f"p {p} db")
