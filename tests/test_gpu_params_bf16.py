"""bf16 parameters read by the kernels (the reference's default layer dtype; its kernels load W in
the stored dtype and widen it, sparse_pooling/kernels/triton_fused.py:257).

* Through Level1Runtime, a layer whose W and bias are bf16 gives the bits of the same layer run on
  the fp32 widening of those values (bf16 -> fp32 is exact, and the arithmetic after the load is
  the same), for every pooling kind and both dX kernels; and it matches the float64 oracle fed
  the widened values (conftest.assert_parity's fp32 bar).
* Through the layer (dtype=torch.bfloat16, the reference's default), the kernels receive the
  parameter tensors themselves: no fp32 copy of W or bias is made per call.
* GELU neurons through the layer: forward, dX, dW, db against the oracle.
"""
import ctypes

import numpy as np
import pytest
import torch

from conftest import assert_parity, gpu_available, rel_err

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

from granulelayer_amd import LevelSpec, PhysicalPlan, SparsePoolingLayer  # noqa: E402
from granulelayer_amd.autograd import Level1Runtime  # noqa: E402
from granulelayer_amd.backend import HipBackend  # noqa: E402
from oracle import oracle as O  # noqa: E402

DEV = "cuda"

# D, H, G, K, B: dX by dx_kernel (long segments: S K 8 >= 64 D) and by dx_dma_kernel (short)
CASES = [(1024, 65536, 64, 8, 300), (2048, 40000, 40, 8, 70), (96, 5000, 7, 16, 33)]
POOLS = [("sum", "relu"), ("mean", "gelu"), ("max", "identity"), ("topk_mean", "gelu"), ("logmeanexp", "relu")]


def _case(D, H, G, K, B, seed=0):
    from test_gpu_parity import make_case

    L, idx, w, b, x, dy = make_case(D, H, G, K, B, seed=seed, bias_std=0.3)
    return L, idx, w.to(torch.bfloat16), b.to(torch.bfloat16), x, dy


def _run(rt, x, w, b, dy, pool):
    track = pool in ("max", "topk_mean")
    out = rt.forward(x, w, b, track_ids=track)
    dw = torch.zeros(rt.layout.weight_shape, device=DEV)
    db = torch.zeros(rt.layout.bias_shape, device=DEV)
    dx = rt.backward(x, w, b, dy, out, "save_winners" if track else "minimal_stats", dw, db)
    torch.cuda.synchronize()
    return out["pre"], dx, dw, db


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}")
@pytest.mark.parametrize("pool,act", POOLS, ids=lambda v: str(v))
def test_bf16_parameters_give_the_bits_of_their_fp32_widening(case, pool, act):
    L, idx, wb, bb, x, dy = _case(*case)
    kw = {"k": 8} if pool == "topk_mean" else ({"temperature": 0.7} if pool == "logmeanexp" else {})
    rt = Level1Runtime(L, idx.to(DEV), LevelSpec(pool, activation=act, **kw), PhysicalPlan())
    xd, dyd = x.to(DEV), dy.to(DEV)
    got = _run(rt, xd, wb.to(DEV), bb.to(DEV), dyd, pool)
    want = _run(rt, xd, wb.float().to(DEV), bb.float().to(DEV), dyd, pool)
    for name, g, e in zip(("pre", "dX", "dW", "db"), got, want):
        assert torch.equal(g, e), f"{name} differs between bf16 parameters and their fp32 widening"
    if pool in ("sum", "mean"):  # the oracle on the bf16-exact values
        K = L.fan_in
        fi, fw, fb = idx.reshape(-1, K).numpy(), wb.float().reshape(-1, K).numpy(), bb.float().reshape(-1).numpy()
        counts = L.counts_tensor("cpu").numpy()
        pre, mag = O.forward(x.numpy(), fi, fw, fb, counts, L.slots_per_group, act, pool, with_mag=True)
        assert_parity(got[0].cpu().numpy(), pre, mag, what="pre")
        wdW, wdb, wdX, bnd = O.backward(x.numpy(), fi, fw, fb, counts, L.slots_per_group, dy.numpy(), act, pool,
                                        with_bounds=True)
        (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
        assert_parity(got[1].cpu().numpy(), wdX, mX, uX, what="dX")
        assert_parity(got[2].cpu().numpy().reshape(-1, K), wdW, mW, uW, what="dW")
        assert_parity(got[3].cpu().numpy().reshape(-1), wdb, mb, ub, what="db")


def _record_launches(monkeypatch):
    """The GlFwdArgs / GlBwdArgs of every gl_fwd / gl_bwd call, as the backend passes them."""
    be = HipBackend.get()
    seen = []
    call = be.lib.call

    def spy(name, *args):
        if name in ("gl_fwd", "gl_bwd"):
            a = args[0]._obj
            seen.append((name, a.W, a.bias, a.w_dtype))
        return call(name, *args)

    monkeypatch.setattr(be.lib, "call", spy)
    return seen


def test_bf16_layer_passes_its_parameters_without_a_copy(monkeypatch):
    from granulelayer_amd import _native as N

    lay = SparsePoolingLayer(512, 20000, 20, shared_neurons=None, pooling="mean", dtype=torch.bfloat16, device=DEV,
                             seed=3, bias_std=0.2)
    assert lay.weight.dtype == torch.bfloat16 and lay.bias.dtype == torch.bfloat16
    lay.enable_main_grad()
    seen = _record_launches(monkeypatch)
    x = torch.randn(40, 512, device=DEV).requires_grad_(True)
    y = lay(x)
    y.backward(torch.randn_like(y))
    torch.cuda.synchronize()
    assert [s[0] for s in seen] == ["gl_fwd", "gl_bwd"]
    for _, wp, bp, code in seen:
        assert wp == lay.weight.data_ptr() and bp == lay.bias.data_ptr() and code == N.GL_DTYPE_BF16
    # the layer's result is the reference's: x rounded to bf16, W and b as stored (bf16), fp32 math
    L = lay.layout
    K = L.fan_in
    fi = lay.indices.cpu().reshape(-1, K).numpy()
    fw = lay.weight.detach().float().cpu().reshape(-1, K).numpy()
    fb = lay.bias.detach().float().cpu().reshape(-1).numpy()
    xn = x.detach().to(torch.bfloat16).float().cpu().numpy()
    pre, mag = O.forward(xn, fi, fw, fb, L.counts_tensor("cpu").numpy(), L.slots_per_group, "relu", "mean",
                         with_mag=True)
    assert_parity(y.detach().cpu().numpy(), pre, mag, what="bf16 layer y")


@pytest.mark.parametrize("pooling", [{"type": "mean", "activation": "gelu"}, {"type": "sum", "activation": "gelu"},
                                     {"type": "max", "activation": "gelu"}])
def test_gelu_layer_matches_oracle(pooling):
    lay = SparsePoolingLayer(256, 12000, 12, shared_neurons=None, pooling=pooling, dtype=torch.float32, device=DEV,
                             seed=5, bias_std=0.3)
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(48, 256, generator=gen).to(DEV).requires_grad_(True)
    dy = torch.randn(48, 12, generator=gen).to(DEV)
    y = lay(x)
    y.backward(dy)
    L = lay.layout
    K = L.fan_in
    fi = lay.indices.cpu().reshape(-1, K).numpy()
    fw = lay.weight.detach().cpu().reshape(-1, K).numpy()
    fb = lay.bias.detach().cpu().reshape(-1).numpy()
    counts = L.counts_tensor("cpu").numpy()
    xn = x.detach().cpu().numpy()
    pool = pooling["type"]
    if pool == "max":  # y = relu(max gelu(z)) (the reference's default max out-activation)
        pre, _, gap = O.forward_max(xn, fi, fw, fb, counts, L.slots_per_group, "gelu")
        want_y = np.maximum(pre, 0.0)
        assert gap.min() > 2e-6
        g_pre = dy.cpu().numpy() * (pre > 0)
        dW, db, dX = O.backward(xn, fi, fw, fb, counts, L.slots_per_group, g_pre.astype(np.float32), "gelu", "max")
    else:
        want_y = O.forward(xn, fi, fw, fb, counts, L.slots_per_group, "gelu", pool)
        dW, db, dX = O.backward(xn, fi, fw, fb, counts, L.slots_per_group, dy.cpu().numpy(), "gelu", pool)
    for name, got, want in (("y", y.detach(), want_y), ("dX", x.grad, dX),
                            ("dW", lay.weight.grad.reshape(-1, K), dW), ("db", lay.bias.grad.reshape(-1), db)):
        e = rel_err(got.cpu().numpy(), want)
        assert e < 2e-5, f"{name}: rel_err {e:.2e}"
    assert lay.last_info["forward_backend"] == "hip" and lay.last_info["backward_backend"] == "hip"
