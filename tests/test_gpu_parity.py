"""Parity of the HIP path (through the C ABI) with the CPU oracle on identical seeded inputs.

fp32 bar (conftest.assert_parity): |got - want| <= 1e-6 + 1e-5 * mag (+ the contribution of relu
masks an fp32 z may decide either way) elementwise, mag being the oracle's sum of |terms| of that
output, and a whole-tensor relative error <= 1e-5 (north star: rel 1e-5 / abs 1e-6);
integer / layout outputs: bit-exact.  The oracle accumulates in float64.
"""
import numpy as np
import pytest
import torch

from conftest import assert_close, assert_parity, gpu_available, rel_err

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

from granulelayer_amd import LevelSpec, PhysicalPlan, SparseLayout, SparsePoolingLayer, init_parameters  # noqa: E402
from granulelayer_amd.autograd import Level1Runtime  # noqa: E402
from granulelayer_amd.backend import HipBackend  # noqa: E402
from oracle import oracle as O  # noqa: E402

DEV = "cuda"


def make_case(D, H, G, K, B, seed=0, x_dtype=torch.float32, bias_std=0.3):
    L = SparseLayout(D, H, G, K, 8, False)
    idx, w, b = init_parameters(L, "cpu", torch.float32, seed=seed, bias_std=bias_std)
    gen = torch.Generator().manual_seed(seed + 1000)
    x = torch.randn(B, D, generator=gen).to(x_dtype)
    dy = torch.randn(B, G, generator=gen)
    return L, idx, w, b, x, dy


def flat(L, idx, w, b):
    K = L.fan_in
    return idx.reshape(-1, K).numpy(), w.reshape(-1, K).numpy(), b.reshape(-1).numpy()


def runtime(L, idx, pool, act):
    return Level1Runtime(L, idx.to(DEV), LevelSpec(pool, activation=act), PhysicalPlan())


FWD_CASES = [
    # D, H, G, K, B, x dtype
    (64, 3000, 8, 8, 1, torch.float32),
    (64, 3000, 8, 8, 37, torch.float32),
    (128, 4099, 16, 8, 130, torch.float32),
    (1024, 20011, 16, 8, 64, torch.bfloat16),
    (1024, 65536, 64, 8, 256, torch.float32),
    (96, 5000, 7, 16, 33, torch.float32),
    (4096, 16384, 16, 8, 8, torch.float32),
]


@pytest.mark.parametrize("case", FWD_CASES, ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}{str(c[5])[6:]}")
@pytest.mark.parametrize("pool,act", [("mean", "relu"), ("sum", "relu"), ("mean", "identity"), ("sum", "identity"),
                                      ("mean", "gelu"), ("sum", "gelu")])
def test_forward_matches_oracle(case, pool, act):
    D, H, G, K, B, xdt = case
    L, idx, w, b, x, _ = make_case(D, H, G, K, B, x_dtype=xdt)
    rt = runtime(L, idx, pool, act)
    pre = rt.forward(x.to(DEV), w.to(DEV), b.to(DEV))["pre"].cpu().numpy()
    fi, fw, fb = flat(L, idx, w, b)
    want, mag = O.forward(x.float().numpy(), fi, fw, fb, L.counts_tensor("cpu").numpy(), L.slots_per_group, act, pool,
                          with_mag=True)
    assert_parity(pre, want, mag, what=f"pre {pool}/{act}")
    assert rt.last_info["forward_backend"] == "hip"


BWD_CASES = [
    (64, 3000, 8, 8, 64, torch.float32),
    (128, 4099, 16, 8, 37, torch.float32),
    (1024, 20011, 16, 8, 64, torch.bfloat16),
    (96, 5000, 7, 16, 33, torch.float32),
    (1024, 65536, 64, 8, 300, torch.float32),
    (2048, 40000, 40, 8, 1100, torch.float32),
]


@pytest.mark.parametrize("case", BWD_CASES, ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}{str(c[5])[6:]}")
@pytest.mark.parametrize("pool,act", [("mean", "relu"), ("sum", "relu"), ("sum", "identity"), ("mean", "gelu"),
                                      ("sum", "gelu")])
def test_backward_matches_oracle(case, pool, act):
    D, H, G, K, B, xdt = case
    L, idx, w, b, x, dy = make_case(D, H, G, K, B, x_dtype=xdt)
    rt = runtime(L, idx, pool, act)
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(x.to(DEV), w.to(DEV), b.to(DEV), dy.to(DEV), {}, "minimal_stats", dw, db).cpu().numpy()
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    wdW, wdb, wdX, bnd = O.backward(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group, dy.numpy(), act, pool,
                                    with_bounds=True)
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_parity(dx, wdX, mX, uX, what="dX")
    assert_parity(dw.cpu().numpy().reshape(-1, K), wdW, mW, uW, what="dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, ub, what="db")
    # padded slots receive no gradient
    valid = L.valid_mask("cpu").reshape(-1).numpy()
    assert not dw.cpu().numpy().reshape(-1, K)[~valid].any()


def make_window_case(D, H, G, K, B, width, seed=0, x_dtype=torch.float32):
    """The C3 index structure: every pool draws its inputs from one contiguous window of `width`
    inputs at a seeded offset (padded slots keep index 0)."""
    from granulelayer_amd.layout import sample_distinct

    L, idx, w, b, x, dy = make_case(D, H, G, K, B, seed=seed, x_dtype=x_dtype)
    S = L.slots_per_group
    gen = torch.Generator().manual_seed(seed + 7)
    off = torch.randint(0, D - width + 1, (G,), generator=gen)
    rec = sample_distinct(G * S, width, K, gen, "cpu").to(torch.int32) + off.repeat_interleave(S)[:, None].to(torch.int32)
    rec[~L.valid_mask("cpu").reshape(-1)] = 0
    return L, rec.view(L.index_shape).to(idx.dtype), w, b, x, dy


# (D, H, G, K, B, window): pools of 1024 (4 per forward workgroup), of 300 (8 per workgroup), K = 16;
# 300 tokens: dX in 256-token slices, by dx_kernel with the windows (long segments) and by
# dx_dma_kernel without them (segments of 32 edges)
WIN_CASES = [(2048, 8192, 8, 8, 37, 256), (1536, 4800, 16, 8, 70, 120), (2048, 2048, 4, 16, 33, 200),
             (2048, 8192, 8, 8, 300, 256)]


@pytest.mark.parametrize("act", ["relu", "identity"])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("case", WIN_CASES, ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}w{c[5]}")
def test_window_staging_matches_full_staging_and_oracle(case, x_dtype, act):
    """Pool-window staging (gl_window_build_host) runs the window kernels and gives bit-identical
    results to full-width staging, within the oracle's bar.  bf16 X stages 4 raw bf16 tokens per
    8-byte input (windows from an even input) in the forward, and in the dW pass of identity neurons
    (and of ReLU neurons with the forward's bits, test_gpu_relu_bits.py); fp32 X 16-byte inputs."""
    from granulelayer_amd import _native as N

    D, H, G, K, B, width = case
    L, idx, w, b, x, dy = make_window_case(D, H, G, K, B, width, x_dtype=x_dtype)
    be = HipBackend.get()
    outs = {}
    try:
        for ws in (True, False):
            be.window_staging = ws
            rt = runtime(L, idx, "sum", act)
            dw = torch.zeros(L.weight_shape, device=DEV)
            db = torch.zeros(L.bias_shape, device=DEV)
            with N.KernelTrace() as tr:
                pre = rt.forward(x.to(DEV), w.to(DEV), b.to(DEV))["pre"]
                dx = rt.backward(x.to(DEV), w.to(DEV), b.to(DEV), dy.to(DEV), {}, "minimal_stats", dw, db)
            names = set(tr.times_ms())
            want = {"fwd_kernel_win", "bwd_w_kernel_win"} if ws else {"fwd_kernel", "bwd_w_kernel"}
            if B > 128:
                want.add("dx_kernel" if ws else "dx_dma_kernel")
            assert want <= names, f"window_staging={ws}: ran {sorted(names)}"
            outs[ws] = [t.cpu() for t in (pre, dw, db, dx)]
    finally:
        be.window_staging = True
    for name, a, c in zip(("pre", "dW", "db", "dX"), outs[True], outs[False]):
        assert torch.equal(a, c), f"{name} differs between window and full staging"
    pre, dw, db, dx = (t.numpy() for t in outs[True])
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    want, mag = O.forward(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group, act, "sum", with_mag=True)
    assert_parity(pre, want, mag, what="pre")
    wdW, wdb, wdX, bnd = O.backward(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group, dy.numpy(), act, "sum",
                                    with_bounds=True)
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_parity(dx, wdX, mX, uX, what="dX")
    assert_parity(dw.reshape(-1, K), wdW, mW, uW, what="dW")
    assert_parity(db.reshape(-1), wdb, mb, ub, what="db")


def _read_edges(edges: torch.Tensor):
    raw = edges.cpu().numpy()
    h = np.frombuffer(raw[:48].tobytes(), dtype=np.int32)
    offs = np.frombuffer(raw[48:80].tobytes(), dtype=np.uint64).astype(np.int64)
    FR, nseg, ne = int(h[7]), int(np.uint32(h[10])), int(np.uint32(h[11]))
    u32 = lambda off, n: np.frombuffer(raw[off:off + 4 * n].tobytes(), dtype=np.uint32)  # noqa: E731
    return dict(magic=int(np.uint32(h[0])), fw=int(h[5]), us=int(h[6]), FR=FR, nseg=nseg, n_edges=ne, seg_ptr=u32(offs[0], FR + 1),
                seg_unit=u32(offs[1], nseg).astype(np.int32), seg_begin=u32(offs[2], nseg + 1), rec=u32(offs[3], ne))


@pytest.mark.parametrize("D,H,G,K", [(64, 3000, 8, 8), (1024, 20011, 16, 8), (96, 5000, 7, 16), (300, 9000, 3, 8)])
def test_edge_list_is_bit_exact(D, H, G, K):
    L, idx, w, b, x, _ = make_case(D, H, G, K, 1)
    rt = runtime(L, idx, "mean", "relu")
    e = _read_edges(HipBackend.get().edges(rt))
    fi, _, _ = flat(L, idx, w, b)
    want = O.xedges(fi, L.counts_tensor("cpu").numpy(), L.slots_per_group, D, e["fw"], e["us"])
    assert (e["fw"], e["us"]) == (8, 1024)
    assert e["magic"] == 0x474C4531
    assert e["n_edges"] == len(want["rec"])
    assert np.array_equal(e["rec"], want["rec"])
    assert np.array_equal(e["seg_ptr"].astype(np.int64), want["seg_ptr"])
    assert np.array_equal(e["seg_unit"], want["seg_unit"])
    assert np.array_equal(e["seg_begin"].astype(np.int64), want["seg_begin"])


@pytest.mark.parametrize("moments", ["fp32", "bf16"])
@pytest.mark.parametrize("n", [10_001, 812_345])
def test_adam_matches_oracle(moments, n):
    gen = torch.Generator().manual_seed(3)
    p = torch.randn(n, generator=gen)
    m = torch.zeros(n)
    v = torch.zeros(n)
    mdt = torch.bfloat16 if moments == "bf16" else torch.float32
    pd, md, vd = p.to(DEV), m.to(mdt).to(DEV), v.to(mdt).to(DEV)
    po, mo, vo = p.numpy().copy(), m.numpy().copy(), v.numpy().copy()
    for t in range(1, 6):
        g = torch.randn(n, generator=gen)
        gd = g.to(DEV)
        HipBackend.get().adam(pd, gd, md, vd, 1e-2, 0.9, 0.999, 1e-8, 0.1, 1 - 0.9 ** t, 1 - 0.999 ** t)
        O.adam(po, g.numpy().copy(), mo, vo, 1e-2, 0.9, 0.999, 1e-8, 0.1, t, moments_bf16=(moments == "bf16"))
        assert float(gd.abs().max()) == 0.0, "fused zero_grad"
    assert_close(pd.cpu().numpy(), po, what="p")
    assert_close(md.float().cpu().numpy(), mo, what="m")
    assert_close(vd.float().cpu().numpy(), vo, what="v")
    exact = float((pd.cpu().numpy() == po).mean())
    print(f"adam {moments} n={n}: {exact * 100:.3f}% of parameters bitwise equal to the oracle")


def test_layer_autograd_and_main_grad():
    D, H, G, K, B = 256, 12000, 12, 8, 48
    lay = SparsePoolingLayer(D, H, G, fan_in=K, shared_neurons=None, pooling="mean", dtype=torch.float32,
                             device=DEV, seed=4, bias_std=0.2)
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(B, D, generator=gen).to(DEV).requires_grad_(True)
    dy = torch.randn(B, G, generator=gen).to(DEV)
    y = lay(x)
    (y * dy).sum().backward()
    L = lay.layout
    fi, fw, fb = flat(L, lay.indices.cpu(), lay.weight.detach().cpu(), lay.bias.detach().cpu())
    counts = L.counts_tensor("cpu").numpy()
    want_y, mag_y = O.forward(x.detach().cpu().numpy(), fi, fw, fb, counts, L.slots_per_group, "relu", "mean",
                              with_mag=True)
    wdW, wdb, wdX, bnd = O.backward(x.detach().cpu().numpy(), fi, fw, fb, counts, L.slots_per_group,
                                    dy.cpu().numpy(), "relu", "mean", with_bounds=True)
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_parity(y.detach().cpu().numpy(), want_y, mag_y, what="y")
    assert_parity(x.grad.cpu().numpy(), wdX, mX, uX, what="dx")
    assert_parity(lay.weight.grad.cpu().numpy().reshape(-1, K), wdW, mW, uW, what="dW")
    assert_parity(lay.bias.grad.cpu().numpy().reshape(-1), wdb, mb, ub, what="db")
    assert lay.last_info["forward_backend"] == "hip" and lay.last_info["backward_backend"] == "hip"
    # main_grad: routed there, accumulates across two backward calls
    lay.enable_main_grad()
    lay.weight.grad = None
    lay(x.detach()).sum().backward()
    g1 = lay.weight.main_grad.clone()
    assert lay.weight.grad is None
    lay(x.detach()).sum().backward()
    assert torch.allclose(lay.weight.main_grad, 2 * g1, rtol=1e-6, atol=1e-9)
    lay.zero_main_grad()
    assert float(lay.weight.main_grad.abs().max()) == 0.0


def test_recompute_is_bitwise_deterministic():
    D, H, G, K, B = 1024, 40000, 16, 8, 96
    L, idx, w, b, x, dy = make_case(D, H, G, K, B, seed=5, bias_std=0.1)
    rt = runtime(L, idx, "mean", "relu")
    args = (x.to(DEV), w.to(DEV), b.to(DEV))
    a = rt.forward(*args)["pre"]
    c = rt.forward(*args)["pre"]
    assert torch.equal(a, c)
    outs = []
    for _ in range(3):
        dw = torch.zeros(L.weight_shape, device=DEV)
        db = torch.zeros(L.bias_shape, device=DEV)
        dx = rt.backward(*args, dy.to(DEV), {}, "minimal_stats", dw, db)
        outs.append((dx, dw, db))
    for o in outs[1:]:
        for p, q in zip(o, outs[0]):
            assert torch.equal(p, q)


def test_inplace_param_update_between_fwd_and_bwd_is_rejected():
    lay = SparsePoolingLayer(64, 3000, 8, shared_neurons=None, pooling="mean", dtype=torch.float32, device=DEV)
    x = torch.randn(4, 64, device=DEV)
    y = lay(x)
    with torch.no_grad():
        lay.weight.add_(1.0)
    with pytest.raises(RuntimeError):
        y.sum().backward()


def _step_extra_bytes(B, H, D=1024):
    lay = SparsePoolingLayer(D, H, H // 1024, shared_neurons=None, pooling="mean", dtype=torch.float32, device=DEV)
    lay.enable_main_grad()
    x = torch.randn(B, D, device=DEV, requires_grad=True)
    lay(x).square().mean().backward()  # builds the persistent input-major edge list
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    lay(x).square().mean().backward()
    torch.cuda.synchronize()
    return torch.cuda.max_memory_allocated() - base


def test_no_hidden_activation_is_materialized():
    """[B, H] in fp32 is B*H*4 bytes; the part of a training step's transient memory that grows
    with H must stay below 1/20 of that (the reference's bound, tests/test_recomputation.py:69-86).
    The backward keeps one activation-mask bit per (token, neuron) -- 1/32 of the fp32 hidden
    tensor -- plus pool-range dX partials that scale with B*D, not H."""
    B = 256
    e1 = _step_extra_bytes(B, 2_097_152)
    e2 = _step_extra_bytes(B, 4_194_304)
    per_neuron = (e2 - e1) / (4_194_304 - 2_097_152)
    assert per_neuron < B * 4 / 20, f"{per_neuron:.1f} transient bytes per neuron suggests materialisation"
    # absolute: the 1/32-size mask plus the B*D-sized dX partials stay far below the hidden tensor
    assert e2 < B * 4_194_304 * 4 / 10, f"peak extra {e2 / 2**20:.0f} MiB"


@pytest.mark.parametrize("cfg,groups", [("C2", 4096), ("C3", 2048), ("C4", 512), ("C5", 2048)])
def test_configs_at_scale_on_sampled_pools(cfg, groups):
    """BASELINE config shapes (B, D, fan-in, pool size, index structure, X dtype) with a few
    thousand pools: the HIP forward, dW and db of 24 random pools against the oracle run on just
    those pools, and the full-layer dX against the oracle's dX of those pools with dY zero on every
    other pool (dX only sums pools whose dY is non-zero)."""
    from granulelayer_amd.synthetic import make_problem

    pr = make_problem(cfg, device="cpu", seed=0, groups=groups)
    L = pr.layout
    S, K = L.slots_per_group, L.fan_in
    rt = Level1Runtime(L, pr.idx.to(DEV), LevelSpec("sum"), PhysicalPlan())
    xd = pr.x.to(DEV)
    pre = rt.forward(xd, pr.w.to(DEV), pr.b.to(DEV))["pre"].cpu().numpy()
    pools = np.sort(np.random.default_rng(0).choice(L.groups, 24, replace=False))
    dy = torch.zeros_like(pr.dy)
    dy[:, pools] = pr.dy[:, pools]
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(xd, pr.w.to(DEV), pr.b.to(DEV), dy.to(DEV), {}, "minimal_stats", dw, db).cpu().numpy()
    sl = np.concatenate([np.arange(g * S, (g + 1) * S) for g in pools])
    fi, fw, fb = flat(L, pr.idx, pr.w, pr.b)
    counts = np.full(len(pools), S, np.int32)
    xn = pr.x.float().numpy()  # bf16 inputs widened exactly, as the kernels do
    want, mag = O.forward(xn, fi[sl], fw[sl], fb[sl], counts, S, "relu", "sum", with_mag=True)
    assert_parity(pre[:, pools], want, mag, what=f"{cfg} pre (sampled pools)")
    wdW, wdb, wdX, bnd = O.backward(xn, fi[sl], fw[sl], fb[sl], counts, S, pr.dy.numpy()[:, pools], "relu", "sum",
                                    with_bounds=True)
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_parity(dw.cpu().numpy().reshape(-1, K)[sl], wdW, mW, uW, what=f"{cfg} dW (sampled pools)")
    assert_parity(db.cpu().numpy().reshape(-1)[sl], wdb, mb, ub, what=f"{cfg} db (sampled pools)")
    assert_parity(dx, wdX, mX, uX, what=f"{cfg} dX (dY on sampled pools)")
    other = np.setdiff1d(np.arange(L.groups), pools)[:64]
    osl = np.concatenate([np.arange(g * S, (g + 1) * S) for g in other])
    assert float(np.abs(dw.cpu().numpy().reshape(-1, K)[osl]).max()) == 0.0, "pools with zero dY get zero dW"


# ---- stored known-answer vectors (tests/golden/make_golden.py) --------------------------------
def _golden(name):
    from pathlib import Path

    with np.load(Path(__file__).resolve().parent / "golden" / "golden_small.npz") as d:
        return {k.split("/", 1)[1]: d[k] for k in d.files if k.startswith(name + "/")}


@pytest.mark.parametrize("name", ["mean_k8", "sum_k8", "sum_k16"])
def test_hip_matches_golden_vectors(name):
    """Forward and backward of the HIP library (arbitrary per-pool counts with padded slots) against
    the stored torch float64 vectors; fp32 bar with the oracle's error scales."""
    from types import SimpleNamespace

    c = _golden(name)
    B, D, G, S, K, pool = (int(v) for v in c["shape"])
    pool = "mean" if pool == 0 else "sum"
    L = SimpleNamespace(groups=G, slots_per_group=S, fan_in=K, input_dim=D, weight_shape=(G * S, K),
                        bias_shape=(G * S,))
    rt = SimpleNamespace(layout=L, level=LevelSpec(pool, activation="relu"), idx=torch.tensor(c["idx"]).to(DEV),
                         counts_i32=torch.tensor(c["counts"]).to(DEV), last_info={})
    hb = HipBackend.get()
    x, w, b = (torch.tensor(c[k]).to(DEV) for k in ("x", "w", "b"))
    pre = hb.forward(rt, x, w, b)["pre"].cpu().numpy()
    _, mag = O.forward(c["x"], c["idx"], c["w"], c["b"], c["counts"], S, "relu", pool, with_mag=True)
    assert_parity(pre, c["pre"], mag, what=f"{name} pre")
    dW = torch.zeros(G * S, K, device=DEV)
    db = torch.zeros(G * S, device=DEV)
    dx = hb.backward(rt, x, w, b, torch.tensor(c["dy"]).to(DEV), {}, dW, db).cpu().numpy()
    _, _, _, bnd = O.backward(c["x"], c["idx"], c["w"], c["b"], c["counts"], S, c["dy"], "relu", pool,
                              with_bounds=True)
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_parity(dx, c["dX"], mX, uX, what=f"{name} dX")
    assert_parity(dW.cpu().numpy(), c["dW"], mW, uW, what=f"{name} dW")
    assert_parity(db.cpu().numpy(), c["db"], mb, ub, what=f"{name} db")


def test_hip_adam_matches_golden_adamw():
    a = _golden("adam")
    lr, b1, b2, eps, wd = (float(v) for v in a["hyper"])
    p = torch.tensor(a["p0"]).to(DEV)
    m = torch.zeros_like(p)
    v = torch.zeros_like(p)
    for t in range(1, 4):
        g = torch.tensor(a["grads"][t - 1]).to(DEV)
        HipBackend.get().adam(p, g, m, v, lr, b1, b2, eps, wd, 1 - b1 ** t, 1 - b2 ** t)
    # torch.optim.AdamW forms 1 - beta in double, the reference in fp32 (see test_golden.py)
    np.testing.assert_allclose(m.cpu().numpy(), a["m"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(v.cpu().numpy(), a["v"], rtol=2e-5, atol=1e-9)
    np.testing.assert_allclose(p.cpu().numpy(), a["p"], rtol=0, atol=3 * lr * 1e-4)


# ---- max pooling (pytorch_reference.py:61-67; winner = first maximum, ties to the smaller slot) ----
MAX_CASES = [
    # D, H, G, K, B, x dtype: ragged pools (padded slots must never win), bf16 X, K = 16, D > 4096
    (64, 3000, 8, 8, 37, torch.float32),
    (1024, 20011, 16, 8, 64, torch.bfloat16),
    (96, 5000, 7, 16, 33, torch.float32),
    (1024, 65536, 64, 8, 260, torch.float32),
    (6000, 9000, 9, 8, 20, torch.float32),
]


def _max_oracle(L, idx, w, b, x, act):
    fi, fw, fb = flat(L, idx, w, b)
    return O.forward_max(x.float().numpy(), fi, fw, fb, L.counts_tensor("cpu").numpy(), L.slots_per_group, act)


@pytest.mark.parametrize("case", MAX_CASES, ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}{str(c[5])[6:]}")
@pytest.mark.parametrize("act", ["identity", "relu", "gelu"])
def test_max_forward_matches_oracle(case, act):
    D, H, G, K, B, xdt = case
    L, idx, w, b, x, _ = make_case(D, H, G, K, B, x_dtype=xdt)
    rt = runtime(L, idx, "max", act)
    out = rt.forward(x.to(DEV), w.to(DEV), b.to(DEV), track_ids=True)
    pre, win = out["pre"].cpu().numpy(), out["winner"].cpu().numpy()
    want, wwin, gap = _max_oracle(L, idx, w, b, x, act)
    # the maximum of fp32 z values: within fp32 rounding of the float64 maximum
    assert_close(pre, want, rtol=1e-5, atol=1e-6, what=f"max pre/{act}")
    # winners bit-exact wherever fp32 cannot swap the two leading neurons
    # fp32 z carries at most ~(K + 1) 2^-24 of its scale: leads above 2e-6 cannot swap
    clear = gap > 2e-6
    assert clear.mean() > 0.99
    assert (win[clear] == wwin[clear]).all(), f"{(win[clear] != wwin[clear]).sum()} winners differ"
    counts = L.counts_tensor("cpu").numpy()
    assert ((win >= 0) & (win < counts[None, :])).all()  # never a padded slot
    # without track_ids only pre is returned, with the same values
    pre2 = rt.forward(x.to(DEV), w.to(DEV), b.to(DEV))
    assert set(pre2) == {"pre"} and torch.equal(pre2["pre"].cpu(), out["pre"].cpu())


@pytest.mark.parametrize("case", MAX_CASES[:4], ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}{str(c[5])[6:]}")
@pytest.mark.parametrize("act", ["identity", "relu", "gelu"])
def test_max_backward_matches_oracle(case, act):
    D, H, G, K, B, xdt = case
    L, idx, w, b, x, dy = make_case(D, H, G, K, B, x_dtype=xdt)
    _, _, gap = _max_oracle(L, idx, w, b, x, act)
    assert gap.min() > 2e-6, "seeded case has a near-tie; the float64 and fp32 winners could differ"
    rt = runtime(L, idx, "max", act)
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    stats = rt.forward(xd, wd, bd, track_ids=True)
    from granulelayer_amd import _native as N

    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    with N.KernelTrace() as tr:
        dx = rt.backward(xd, wd, bd, dy.to(DEV), stats, "save_winners", dw, db).cpu().numpy()
    # the winner-event kernels ran, not the dense dW / dX passes
    names = set(tr.times_ms())
    assert {"max_events_dw_kernel", "max_events_dx_kernel"} <= names and not {"dx_kernel", "dx_dma_kernel"} & names, sorted(names)
    # deterministic: a second backward gives the same bits
    dw2, db2 = torch.zeros_like(dw), torch.zeros_like(db)
    dx2 = rt.backward(xd, wd, bd, dy.to(DEV), stats, "save_winners", dw2, db2).cpu().numpy()
    assert np.array_equal(dx, dx2) and torch.equal(dw, dw2) and torch.equal(db, db2)
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    wdW, wdb, wdX, bnd = O.backward(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group, dy.numpy(), act, "max",
                                    with_bounds=True)
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_parity(dx, wdX, mX, uX, what="max dX")
    assert_parity(dw.cpu().numpy().reshape(-1, K), wdW, mW, uW, what="max dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, ub, what="max db")
    # at most one neuron per (token, pool) has a gradient: db is non-zero on at most B slots per pool
    assert (np.count_nonzero(db.cpu().numpy().reshape(G, -1), axis=1) <= B).all()
    # the ABI refuses a max backward without winners
    with pytest.raises(Exception):
        rt.backward(xd, wd, bd, dy.to(DEV), {}, "save_winners", dw, db)


@pytest.mark.parametrize("policy", ["save_winners", "minimal_stats"])
def test_max_layer_autograd_policies(policy):
    """SparsePoolingLayer with max pooling (defaults: identity activation, relu out-activation, so
    y = relu(max z)): save_winners keeps the forward's winners, minimal_stats recomputes them in
    backward (autograd.py:246-258); both give the oracle's gradients."""
    D, H, G, K, B = 256, 12000, 12, 8, 40
    lay = SparsePoolingLayer(D, H, G, fan_in=K, shared_neurons=None, pooling="max", checkpoint_policy=policy,
                             dtype=torch.float32, device=DEV, seed=6, bias_std=0.2)
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(B, D, generator=gen).to(DEV).requires_grad_(True)
    dy = torch.randn(B, G, generator=gen).to(DEV)
    y = lay(x)
    (y * dy).sum().backward()
    L = lay.layout
    fi, fw, fb = flat(L, lay.indices.cpu(), lay.weight.detach().cpu(), lay.bias.detach().cpu())
    counts = L.counts_tensor("cpu").numpy()
    want_pre, _, gap = O.forward_max(x.detach().cpu().numpy(), fi, fw, fb, counts, L.slots_per_group, "identity")
    assert gap.min() > 2e-6 and np.abs(want_pre).min() > 1e-5  # no near-ties, no pre near the relu kink
    g_pre = (dy.cpu().numpy() * (want_pre > 0)).astype(np.float32)  # dL/dpre through the relu out-activation
    wdW, wdb, wdX, bnd = O.backward(x.detach().cpu().numpy(), fi, fw, fb, counts, L.slots_per_group, g_pre,
                                    "identity", "max", with_bounds=True)
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_close(y.detach().cpu().numpy(), np.maximum(want_pre, 0.0), rtol=1e-5, atol=1e-6, what="y")
    assert_parity(x.grad.cpu().numpy(), wdX, mX, uX, what="dx")
    assert_parity(lay.weight.grad.cpu().numpy().reshape(-1, K), wdW, mW, uW, what="dW")
    assert_parity(lay.bias.grad.cpu().numpy().reshape(-1), wdb, mb, ub, what="db")
    assert lay.last_info["recomputed_stats"] == (policy == "minimal_stats")


# ---- top-k mean pooling (pytorch_reference.py:68-77: the k largest raw z, ties to the smaller slot) ----
TOPK_CASES = MAX_CASES[:4]


def _runtime_topk(L, idx, act, k):
    return Level1Runtime(L, idx.to(DEV), LevelSpec("topk_mean", activation=act, k=k), PhysicalPlan())


@pytest.mark.parametrize("case", TOPK_CASES, ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}{str(c[5])[6:]}")
@pytest.mark.parametrize("act,k", [("identity", 1), ("identity", 8), ("relu", 8), ("identity", 64), ("gelu", 8),
                                   ("gelu", 16)])
def test_topk_forward_matches_oracle(case, act, k):
    D, H, G, K, B, xdt = case
    L, idx, w, b, x, _ = make_case(D, H, G, K, B, x_dtype=xdt)
    rt = _runtime_topk(L, idx, act, k)
    out = rt.forward(x.to(DEV), w.to(DEV), b.to(DEV), track_ids=True)
    pre, slots = out["pre"].cpu().numpy(), out["topk_slot"].cpu().numpy()
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    want, wslots, gap = O.forward_topk(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group, k, act)
    assert_close(pre, want, rtol=1e-5, atol=1e-6, what=f"top-{k} pre/{act}")
    # the selected set is bit-exact wherever fp32 cannot move the boundary (lead > 2e-6 of the scale);
    # within the set, near-equal values may be listed in either order
    clear = gap > 2e-6
    assert clear.mean() > 0.99
    assert (np.sort(slots, -1)[clear] == np.sort(wslots, -1)[clear]).all()
    kk = np.minimum(counts, k)
    assert ((slots >= 0).sum(-1) == kk[None, :]).all() and (slots < counts[None, :, None]).all()
    pre2 = rt.forward(x.to(DEV), w.to(DEV), b.to(DEV))
    assert set(pre2) == {"pre"} and torch.equal(pre2["pre"].cpu(), out["pre"].cpu())


@pytest.mark.parametrize("case", TOPK_CASES[:3], ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}{str(c[5])[6:]}")
@pytest.mark.parametrize("act,k", [("identity", 8), ("relu", 4), ("identity", 64), ("gelu", 8)])
def test_topk_backward_matches_oracle(case, act, k):
    """The selection events of the HIP forward, checked against the oracle's backward of the same
    selection (which equals its top-k backward, test_oracle.py), plus determinism."""
    from granulelayer_amd import _native as N

    D, H, G, K, B, xdt = case
    L, idx, w, b, x, dy = make_case(D, H, G, K, B, x_dtype=xdt)
    rt = _runtime_topk(L, idx, act, k)
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    stats = rt.forward(xd, wd, bd, track_ids=True)
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    with N.KernelTrace() as tr:
        dx = rt.backward(xd, wd, bd, dy.to(DEV), stats, "save_winners", dw, db).cpu().numpy()
    names = set(tr.times_ms())
    assert {"max_events_dw_kernel", "max_events_dx_kernel"} <= names and not {"dx_kernel", "dx_dma_kernel"} & names, sorted(names)
    dw2, db2 = torch.zeros_like(dw), torch.zeros_like(db)
    dx2 = rt.backward(xd, wd, bd, dy.to(DEV), stats, "save_winners", dw2, db2).cpu().numpy()
    assert np.array_equal(dx, dx2) and torch.equal(dw, dw2) and torch.equal(db, db2)
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_events(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group,
                                                    dy.numpy(), stats["topk_slot"].cpu().numpy(), act, topk=True)
    assert_parity(dx, wdX, mX, what=f"top-{k} dX")
    assert_parity(dw.cpu().numpy().reshape(-1, K), wdW, mW, what=f"top-{k} dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, what=f"top-{k} db")


@pytest.mark.parametrize("policy", ["save_winners", "minimal_stats"])
def test_topk_layer_autograd_policies(policy):
    """SparsePoolingLayer with top-k mean (k = 8, identity activations): the gradients equal the
    oracle's backward of the layer's own selection, with the slots saved or recomputed."""
    D, H, G, K, B = 256, 12000, 12, 8, 40
    lay = SparsePoolingLayer(D, H, G, fan_in=K, shared_neurons=None, pooling={"type": "topk_mean", "k": 8},
                             checkpoint_policy=policy, dtype=torch.float32, device=DEV, seed=8, bias_std=0.2)
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(B, D, generator=gen).to(DEV).requires_grad_(True)
    dy = torch.randn(B, G, generator=gen).to(DEV)
    y = lay(x)
    (y * dy).sum().backward()
    L = lay.layout
    fi, fw, fb = flat(L, lay.indices.cpu(), lay.weight.detach().cpu(), lay.bias.detach().cpu())
    counts = L.counts_tensor("cpu").numpy()
    want, slots, gap = O.forward_topk(x.detach().cpu().numpy(), fi, fw, fb, counts, L.slots_per_group, 8)
    assert gap.min() > 2e-6  # the seeded case has no near-tie at the selection boundary
    assert_close(y.detach().cpu().numpy(), want, rtol=1e-5, atol=1e-6, what="y")
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_events(x.detach().cpu().numpy(), fi, fw, fb, counts, L.slots_per_group,
                                                    dy.cpu().numpy(), slots, "identity", topk=True)
    assert_parity(x.grad.cpu().numpy(), wdX, mX, what="dx")
    assert_parity(lay.weight.grad.cpu().numpy().reshape(-1, K), wdW, mW, what="dW")
    assert_parity(lay.bias.grad.cpu().numpy().reshape(-1), wdb, mb, what="db")
    assert lay.last_info["recomputed_stats"] == (policy == "minimal_stats")


# two backward token chunks (B > 1024: the event kernels' b0 > 0) and D = 8192 (dX event LDS of 96 KiB)
SEL_EDGE_CASES = [(2048, 8000, 8, 8, 1100, torch.float32), (8192, 6000, 6, 8, 70, torch.bfloat16)]


@pytest.mark.parametrize("case", SEL_EDGE_CASES, ids=lambda c: f"D{c[0]}H{c[1]}G{c[2]}K{c[3]}B{c[4]}{str(c[5])[6:]}")
@pytest.mark.parametrize("pool,k", [("max", 1), ("topk_mean", 8)])
def test_selection_backward_chunks_and_wide_inputs(case, pool, k):
    D, H, G, K, B, xdt = case
    L, idx, w, b, x, dy = make_case(D, H, G, K, B, x_dtype=xdt)
    spec = LevelSpec(pool, activation="relu", k=k) if pool == "topk_mean" else LevelSpec(pool, activation="relu")
    rt = Level1Runtime(L, idx.to(DEV), spec, PhysicalPlan())
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    stats = rt.forward(xd, wd, bd, track_ids=True)
    key = "winner" if pool == "max" else "topk_slot"
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(xd, wd, bd, dy.to(DEV), stats, "save_winners", dw, db).cpu().numpy()
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    xn = x.float().numpy()
    if pool == "max":
        want, _, _ = O.forward_max(xn, fi, fw, fb, counts, L.slots_per_group, "relu")
    else:
        want, _, _ = O.forward_topk(xn, fi, fw, fb, counts, L.slots_per_group, k, "relu")
    assert_close(stats["pre"].cpu().numpy(), want, rtol=1e-5, atol=1e-6, what=f"{pool} pre")
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_events(xn, fi, fw, fb, counts, L.slots_per_group, dy.numpy(),
                                                    stats[key].cpu().numpy(), "relu", topk=pool == "topk_mean")
    assert_parity(dx, wdX, mX, what=f"{pool} dX")
    assert_parity(dw.cpu().numpy().reshape(-1, K), wdW, mW, what=f"{pool} dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, what=f"{pool} db")


@pytest.mark.parametrize("k", [16, 64])
def test_topk_pools_shorter_than_k(k):
    """Pools of 12-13 neurons with k = 16 / 64: every valid neuron is selected (kk = n_g), the padded
    list entries never are, and the slots past kk are -1 (pytorch_reference.py:68-77)."""
    D, H, G, K, B = 64, 100, 8, 8, 21
    L, idx, w, b, x, dy = make_case(D, H, G, K, B)
    rt = _runtime_topk(L, idx, "identity", k)
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    out = rt.forward(xd, wd, bd, track_ids=True)
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    want, wslots, _ = O.forward_topk(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group, k)
    assert (counts < k).all()
    assert_close(out["pre"].cpu().numpy(), want, rtol=1e-5, atol=1e-6, what="pre")
    slots = out["topk_slot"].cpu().numpy()
    assert (np.sort(slots, -1) == np.sort(wslots, -1)).all()  # the whole pool, -1 padding
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(xd, wd, bd, dy.to(DEV), out, "save_winners", dw, db).cpu().numpy()
    wdW, wdb, wdX, bnd = O.backward_topk(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group, dy.numpy(), k,
                                         "identity", with_bounds=True)
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_parity(dx, wdX, mX, uX, what="dX")
    assert_parity(dw.cpu().numpy().reshape(-1, K), wdW, mW, uW, what="dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, ub, what="db")


@pytest.mark.parametrize("act", ["identity", "relu"])
def test_topk_ranked_tiles_equal_the_rounds(act):
    """k <= 8 runs the ranked tile (a lower bound of the k-th largest value, the candidates at or
    above it ranked in an LDS list), k = 16 the extraction rounds: on the same layer the top-8 slots,
    best first, are the first 8 of the top-16 list, bit for bit, and pre matches the oracle."""
    D, H, G, K, B = 1024, 65536, 64, 8, 37
    L, idx, w, b, x, _ = make_case(D, H, G, K, B)
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    s8 = _runtime_topk(L, idx, act, 8).forward(xd, wd, bd, track_ids=True)
    s16 = _runtime_topk(L, idx, act, 16).forward(xd, wd, bd, track_ids=True)
    assert torch.equal(s8["topk_slot"].cpu(), s16["topk_slot"].cpu()[..., :8])
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    want, _, _ = O.forward_topk(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group, 8, act)
    assert_close(s8["pre"].cpu().numpy(), want, rtol=1e-5, atol=1e-6, what="top-8 pre")


def test_topk_tied_levels_rank_token_by_token():
    """z on 8 levels (zero weights, each neuron's bias one of 8 values): ~32 of a chunk's 256
    candidates share the top level, so a token's list holds 17-64 keys and the ranked tile ranks
    token by token (not 4 tokens at once); the ties go to the smaller slots. The top-8 slots
    equal the first 8 of the rounds' top-16 list, and pre matches the oracle."""
    D, H, G, K, B = 256, 32768, 32, 8, 9
    L, idx, w, b, x, _ = make_case(D, H, G, K, B)
    w = torch.zeros_like(w)
    gen = torch.Generator().manual_seed(7)
    b = (torch.randint(0, 8, b.shape, generator=gen).float() * 0.125).contiguous()
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    s8 = _runtime_topk(L, idx, "identity", 8).forward(xd, wd, bd, track_ids=True)
    s16 = _runtime_topk(L, idx, "identity", 16).forward(xd, wd, bd, track_ids=True)
    assert torch.equal(s8["topk_slot"].cpu(), s16["topk_slot"].cpu()[..., :8])
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    want, wslots, _ = O.forward_topk(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group, 8, "identity")
    assert_close(s8["pre"].cpu().numpy(), want, rtol=1e-6, atol=1e-7, what="top-8 pre")
    assert (np.sort(s8["topk_slot"].cpu().numpy(), -1) == np.sort(wslots, -1)).all()


def test_topk_all_tied_takes_the_smallest_slots():
    """Every z of a pool equal (zero weights, one bias value): all 256 candidates of a chunk reach
    the ranked tile's bound, more than its 64-entry lists hold, so the tile takes the rounds; the
    top-8 are the 8 smallest slots of each pool (the reference's stable descending sort)."""
    D, H, G, K, B = 256, 8192, 8, 8, 9
    L, idx, w, b, x, _ = make_case(D, H, G, K, B)
    w = torch.zeros_like(w)
    b = torch.full_like(b, 0.25)
    out = _runtime_topk(L, idx, "identity", 8).forward(x.to(DEV), w.to(DEV), b.to(DEV), track_ids=True)
    slots = out["topk_slot"].cpu().numpy()
    assert (np.sort(slots, -1) == np.arange(8)[None, None, :]).all()
    assert torch.equal(out["pre"].cpu(), torch.full((B, G), 0.25))


@pytest.mark.parametrize("pooling", ["sum", "mean", "max", {"type": "topk_mean", "k": 8}],
                         ids=["sum", "mean", "max", "topk8"])
def test_empty_batch(pooling):
    """B = 0 through the layer: an empty [0, G] output, an empty dX and zero parameter gradients
    (the C-ABI refuses B < 1; the backend answers an empty batch without launching)."""
    D, H, G, K = 128, 3000, 6, 8
    lay = SparsePoolingLayer(D, H, G, fan_in=K, shared_neurons=None, pooling=pooling,
                             checkpoint_policy="save_winners", dtype=torch.float32, device=DEV, seed=3)
    x = torch.zeros(0, D, device=DEV, requires_grad=True)
    y = lay(x)
    assert tuple(y.shape) == (0, G)
    y.sum().backward()
    assert tuple(x.grad.shape) == (0, D)
    assert not lay.weight.grad.any() and not lay.bias.grad.any()


@pytest.mark.parametrize("k", [8, 64])
def test_topk_largest_pools(k):
    """Pools of 4000 slots: 16 chunks per pool, the most the top-k finalize merges (larger pools
    are refused), through the generic finalize; forward and the event backward against the oracle."""
    D, H, G, K, B = 64, 12000, 3, 8, 9
    L, idx, w, b, x, dy = make_case(D, H, G, K, B)
    assert L.slots_per_group > 15 * 256
    rt = _runtime_topk(L, idx, "identity", k)
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    out = rt.forward(xd, wd, bd, track_ids=True)
    fi, fw, fb = flat(L, idx, w, b)
    counts = L.counts_tensor("cpu").numpy()
    want, wslots, gap = O.forward_topk(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group, k)
    assert_close(out["pre"].cpu().numpy(), want, rtol=1e-5, atol=1e-6, what=f"top-{k} pre")
    slots = out["topk_slot"].cpu().numpy()
    clear = gap > 2e-6
    assert clear.mean() > 0.9
    assert (np.sort(slots, -1)[clear] == np.sort(wslots, -1)[clear]).all()
    dw = torch.zeros(L.weight_shape, device=DEV)
    db = torch.zeros(L.bias_shape, device=DEV)
    dx = rt.backward(xd, wd, bd, dy.to(DEV), out, "save_winners", dw, db).cpu().numpy()
    wdW, wdb, wdX, (mW, mb, mX) = O.backward_events(x.float().numpy(), fi, fw, fb, counts, L.slots_per_group,
                                                    dy.numpy(), slots, "identity", topk=True)
    assert_parity(dx, wdX, mX, what="dX")
    assert_parity(dw.cpu().numpy().reshape(-1, K), wdW, mW, what="dW")
    assert_parity(db.cpu().numpy().reshape(-1), wdb, mb, what="db")


@pytest.mark.parametrize("D,H,G,window", [(4096, 200_000, 200, 0), (300, 9000, 7, 0), (2048, 8192, 8, 256),
                                          (64, 3000, 8, 0)])
def test_gpu_setup_builders_equal_the_host_builders(D, H, G, window):
    """The gather schedule and the pool windows built on the GPU (gl_sched_build, gl_window_build)
    are bit-identical to the host builders' (gl_sched_build_host, gl_window_build_host)."""
    from granulelayer_amd import _native as N

    if window:
        L, idx, w, b, x, _ = make_window_case(D, H, G, 8, 1, window)
    else:
        L, idx, w, b, x, _ = make_case(D, H, G, 8, 1)
    rt = runtime(L, idx, "sum", "relu")
    be = HipBackend.get()
    lib = N.library()
    S = L.slots_per_group
    host_sched = lib.sched_build(idx.reshape(-1, 8).numpy(), L.counts_tensor("cpu").numpy(), D, G, S, 8)
    assert np.array_equal(be.schedule(rt).cpu().numpy().view(np.uint32), host_sched)
    lo, width = lib.window_build(idx.reshape(-1, 8).numpy(), L.counts_tensor("cpu").numpy(), D, G, S, 8)
    glo, gwidth = be.windows(rt)
    assert gwidth == width and np.array_equal(glo.cpu().numpy().view(np.uint32), lo)
