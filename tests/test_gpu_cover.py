"""Cover-TopK/16 on the GPU: the HIP selection kernel (gl_cover_select) bit-exact against the
reference's own vectors and against the CPU oracle (oracle/cover.py); the compact layer (one K16
record per 16 neurons, rec_shift 4) against the float64 oracle of the same parameters; energy
restoration; save_packed / load_packed; and the C5 shape at full size."""
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import assert_close, assert_parity, gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

from granulelayer_amd import CoverTopK16Layer  # noqa: E402
from granulelayer_amd import cover_topk16 as CT  # noqa: E402
from oracle import cover as OC  # noqa: E402
from oracle import oracle as O  # noqa: E402

DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden" / "cover_reference.npz"


def _golden():
    with np.load(GOLDEN) as z:
        d = {k: z[k] for k in z.files}
    names = sorted({k.split("/")[0] for k in d})
    return [(n, {k.split("/", 1)[1]: v for k, v in d.items() if k.startswith(n + "/")}) for n in names]


@pytest.mark.parametrize("name,case", _golden(), ids=lambda c: c if isinstance(c, str) else "")
def test_selection_kernel_matches_reference_vectors(name, case):
    H, G, C, seed = (int(v) for v in case["shape"])
    L = CT.EnvelopeLayout(4096, H, G, 64, C)
    w = torch.from_numpy(case["w_int"].astype(np.float32) / 4096).to(DEV)
    a = CT.feature_importance(w, L).cpu().numpy()
    assert np.array_equal(a, case["importance"]), "float64 importances differ"
    uv = case["valid_groups"]
    env0 = CT.topk_select(torch.from_numpy(case["importance"][uv]).to(DEV), 16).cpu().numpy()
    assert np.array_equal(env0, case["env_topk"])
    out = CT.cover_topk(w, L)
    assert np.array_equal(out["env"].cpu().numpy()[uv], case["env_cover"])
    rv = L.record_counts("cpu").numpy() > 0
    assert np.array_equal(out["missing0"].cpu().numpy()[rv], case["missing0"])
    assert np.array_equal(out["swaps"].cpu().numpy()[rv], case["swaps"])
    assert np.array_equal(out["loss"].cpu().numpy()[rv], case["loss"]), "energy loss (float64, swap order) differs"


def _envelope(D, H, G, C, seed, quant=None):
    L = CT.EnvelopeLayout(D, H, G, 64, C)
    gen = torch.Generator().manual_seed(seed)
    w = torch.randn(L.weight_shape, generator=gen) / 8
    if quant:  # coarse values: many importance ties
        w = torch.round(w * quant) / quant
    valid = L.valid_mask("cpu")
    w = w * valid[..., None]
    b = torch.randn(L.bias_shape, generator=gen) * 0.2 * valid
    from granulelayer_amd.layout import sample_distinct

    cand = sample_distinct(G * L.blocks_per_group, D, 64, gen, "cpu").to(torch.int32).view(L.index_shape)
    return L, w, b, cand


@pytest.mark.parametrize("C,quant", [(256, None), (64, 4), (128, 2), (16, None)])
def test_selection_kernel_matches_oracle(C, quant):
    D, G = 300, 5
    H = G * (3 * C - 5)  # two full records and a partial one whose last group is partial, per output
    L, w, b, cand = _envelope(D, H, G, C, seed=C, quant=quant)
    gpb = C // 16
    nv = L.valid_mask("cpu").reshape(-1, 16).sum(1).numpy()
    if C == 16:  # one group per record: m k < 64, infeasible for the repair
        with pytest.raises(ValueError, match="infeasible"):
            CT.cover_topk(w.to(DEV), L, cand.to(DEV))
        return
    env, a, m0, sw, lo = OC.select(w.numpy().reshape(-1, 16, 64), nv, gpb, 16, repair=True)
    out = CT.cover_topk(w.to(DEV), L, cand.to(DEV))
    valid = nv > 0
    assert np.array_equal(out["env"].cpu().numpy()[valid], env[valid])
    assert np.array_equal(out["env"].cpu().numpy()[~valid], np.tile(np.arange(16), (int((~valid).sum()), 1)))
    assert np.array_equal(out["swaps"].cpu().numpy(), sw) and np.array_equal(out["missing0"].cpu().numpy(), m0)
    assert np.array_equal(out["loss"].cpu().numpy(), lo)
    # kept global inputs and weights
    ci = cand.numpy().reshape(-1, 64).repeat(gpb, 0)
    assert np.array_equal(out["rec_idx"].cpu().numpy(), np.take_along_axis(ci, out["env"].cpu().numpy(), 1))
    wn = w.numpy().reshape(-1, 64)
    e16 = out["env"].cpu().numpy().repeat(16, 0)
    assert np.array_equal(out["W_out"].cpu().numpy(), np.take_along_axis(wn, e16, 1))


def _layer_oracle(lay, x, dy, pool="mean"):
    """Oracle forward / backward of the compact layer, its records expanded per neuron (Mode A, K 16)."""
    L = lay.layout
    S = L.slots_per_group
    idx = lay.indices.cpu().numpy().reshape(-1, 16).repeat(16, 0)  # [G S, 16]
    w = lay.weight.detach().cpu().numpy().reshape(-1, 16)
    b = lay.bias.detach().cpu().numpy().reshape(-1)
    counts = L.counts_tensor("cpu").numpy()
    want, mag = O.forward(x, idx, w, b, counts, S, "relu", pool, with_mag=True)
    dW, db, dX, bnd = O.backward(x, idx, w, b, counts, S, dy, "relu", pool, with_bounds=True)
    return want, mag, dW, db, dX, bnd


@pytest.mark.parametrize("normalization", ["none", "energy"])
def test_compact_layer_matches_oracle(normalization):
    D, G, C, B = 512, 6, 256, 70
    H = G * (C + 9 * 16 + 5)  # a full record and a partial one whose last group is partial
    L, w, b, cand = _envelope(D, H, G, C, seed=3)
    lay = CoverTopK16Layer.from_envelope(w.to(DEV), b.to(DEV), cand.to(DEV), input_dim=D, hidden_dim=H, output_dim=G,
                                         envelope_C=C, normalization=normalization)
    meta = lay.metadata
    assert meta["valid_slots"] == 16 * H and meta["executed"] == dict(K=16, C=16, records_16=int(
        L.valid_mask("cpu").reshape(-1, 16).any(1).sum()))
    # the compact parameters are the selected envelope values (scaled once with energy restoration)
    nv = L.valid_mask("cpu").reshape(-1, 16).sum(1).numpy()
    env, *_ = OC.select(w.numpy().reshape(-1, 16, 64), nv, C // 16, 16, repair=True)
    kept = np.take_along_axis(w.numpy().reshape(-1, 64), env.repeat(16, 0), 1)
    got_w = lay.weight.detach().cpu().numpy().reshape(-1, 16)
    if normalization == "none":
        assert np.array_equal(got_w, kept)
    else:
        wd = w.numpy().reshape(-1, 64).astype(np.float64)
        e, ek = (wd * wd).sum(1), (kept.astype(np.float64) ** 2).sum(1)
        with np.errstate(invalid="ignore"):  # padded neurons: 0 / 0, replaced below
            s = np.minimum(np.sqrt(e / np.maximum(ek, 1e-6 * e)), 8.0)
        s = np.where(e > 0, s, 1.0) * L.valid_mask("cpu").reshape(-1).numpy()
        assert_close(got_w, kept * s[:, None], rtol=2e-6, atol=1e-12, what="energy-restored weights")
        assert meta["normalization"]["treatment"] == "energy"
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(B, D, generator=gen)
    dy = torch.randn(B, G, generator=gen)
    xd = x.to(DEV).requires_grad_(True)
    lay.enable_main_grad()
    y = lay(xd)
    y.backward(dy.to(DEV))
    want, mag, dW, db, dX, bnd = _layer_oracle(lay, x.numpy(), dy.numpy())
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_parity(y.detach().cpu().numpy(), want, mag, what="y")
    assert_parity(xd.grad.cpu().numpy(), dX, mX, uX, what="dX")
    assert_parity(lay.weight.main_grad.cpu().numpy().reshape(-1, 16), dW, mW, uW, what="dW")
    assert_parity(lay.bias.main_grad.cpu().numpy().reshape(-1), db, mb, ub, what="db")
    assert lay.last_info["forward_backend"] == "hip"


def test_packed_round_trip(tmp_path):
    D, G, C, B = 256, 4, 128, 33
    H = G * 2 * C
    L, w, b, cand = _envelope(D, H, G, C, seed=9)
    lay = CoverTopK16Layer.from_envelope(w.to(DEV), b.to(DEV), cand.to(DEV), input_dim=D, hidden_dim=H, output_dim=G,
                                         envelope_C=C)
    x = torch.randn(B, D, device=DEV)
    y = lay(x)
    info = lay.save_packed(tmp_path / "ct16.pt")
    back = CoverTopK16Layer.load_packed(tmp_path / "ct16.pt", device=DEV)
    assert torch.equal(back(x), y)
    assert back.metadata == lay.metadata and info["fingerprints"] == back.immutable_fingerprints()
    blob = torch.load(tmp_path / "ct16.pt", weights_only=True)
    blob["state"]["indices"][0, 0, 0] += 1  # a changed support must be refused
    torch.save(blob, tmp_path / "bad.pt")
    with pytest.raises(ValueError, match="fingerprints"):
        CoverTopK16Layer.load_packed(tmp_path / "bad.pt", device=DEV)


def test_cover_topk16_at_the_c5_shape():
    """BASELINE configs[4]'s shape with Cover-TopK/16 records: N = 50,331,648 neurons in pools of
    512 (G = 98,304), D = 4096, B = 512, a C256 envelope of 64 candidates uniform in [0, 4096) with
    weights N(0, 1/16); selection of all 196,608 records, then forward and backward of the whole
    compact layer against the oracle on 12 pools (dY zero elsewhere)."""
    D, G, C, B, pool = 4096, 98_304, 256, 512, 512
    H = G * pool
    L = CT.EnvelopeLayout(D, H, G, 64, C)
    gen = torch.Generator(device=DEV).manual_seed(0)
    w = torch.randn(L.weight_shape, generator=gen, device=DEV) / 4
    b = torch.zeros(L.bias_shape, device=DEV)
    from granulelayer_amd.layout import sample_distinct

    cand = torch.empty((G * L.blocks_per_group, 64), dtype=torch.int32, device=DEV)
    for s in range(0, cand.shape[0], 1 << 16):
        e = min(s + (1 << 16), cand.shape[0])
        cand[s:e] = sample_distinct(e - s, D, 64, gen, DEV).to(torch.int32)
    lay = CoverTopK16Layer.from_envelope(w, b, cand.view(L.index_shape), input_dim=D, hidden_dim=H, output_dim=G,
                                         envelope_C=C, pooling="sum")
    del w
    st = lay.metadata["support_stats"]
    print(f"C5 Cover-TopK/16: {st}, selection {lay.metadata['construction_seconds']['selection']:.2f} s")
    assert st["swaps"] == st["missing0"] > 0
    x = torch.randn(B, D, generator=gen, device=DEV)
    pools = np.sort(np.concatenate([[0, G - 1], np.random.default_rng(0).choice(G - 2, 10, replace=False) + 1]))
    sel = torch.from_numpy(pools).to(DEV)
    dy = torch.zeros(B, G, device=DEV)
    dy[:, sel] = torch.randn(B, len(pools), generator=gen, device=DEV)
    xd = x.clone().requires_grad_(True)
    lay.enable_main_grad()
    y = lay(xd)
    y.backward(dy)
    S = lay.layout.slots_per_group
    rows = torch.cat([torch.arange(g * S // 16, (g + 1) * S // 16, device=DEV) for g in pools.tolist()])
    idx = lay.indices.view(-1, 16)[rows].cpu().numpy().repeat(16, 0)
    wk = lay.weight.detach().view(-1, 16, 16)[rows].cpu().numpy().reshape(-1, 16)
    bk = lay.bias.detach().view(-1, 16)[rows].cpu().numpy().reshape(-1)
    counts = np.full(len(pools), pool, np.int32)
    xn = x.cpu().numpy()
    want, mag = O.forward(xn, idx, wk, bk, counts, S, "relu", "sum", with_mag=True)
    assert_parity(y.detach()[:, sel].cpu().numpy(), want, mag, what="C5 Cover-TopK/16 y (sampled pools)")
    dW, db, dX, bnd = O.backward(xn, idx, wk, bk, counts, S, dy[:, sel].cpu().numpy(), "relu", "sum",
                                 with_bounds=True)
    (mW, mb, mX), (uW, ub, uX) = bnd["mag"], bnd["unc"]
    assert_parity(xd.grad.cpu().numpy(), dX, mX, uX, what="C5 Cover-TopK/16 dX")
    assert_parity(lay.weight.main_grad.view(-1, 16, 16)[rows].cpu().numpy().reshape(-1, 16), dW, mW, uW, what="dW")
