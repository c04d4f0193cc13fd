"""FusedAdamW with bf16 parameters on the GPU (sparse_pooling/optim.py:5-9, 26-64): nearest-even
rounding, fp32 master weights and stochastic rounding (Philox noise of tl.randint(seed, element))
against the oracle (oracle.adam_bf16), bit for bit, over three steps, with fp32 and bf16 moments
and a length that is not a multiple of the kernel's 4-element vectors; and the optimizer's seed
sequence (one launch per parameter and step, the reference's _seed counter) and master state."""
import numpy as np
import pytest
import torch

from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

from granulelayer_amd import FusedAdamW  # noqa: E402
from granulelayer_amd.backend import backend_for  # noqa: E402
from oracle import oracle as O  # noqa: E402

DEV = "cuda"
HP = dict(lr=1e-2, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).copy()


@pytest.mark.parametrize("mode", ["nearest", "master", "stochastic"])
@pytest.mark.parametrize("moments", [torch.float32, torch.bfloat16])
def test_gl_adam_bf16_matches_oracle(mode, moments):
    n = 1_000_003
    gen = torch.Generator().manual_seed(4)
    p = (torch.randn(n, generator=gen) * 0.3).to(torch.bfloat16)
    pd = p.to(DEV)
    md = torch.zeros(n, dtype=moments, device=DEV)
    vd = torch.zeros(n, dtype=moments, device=DEV)
    master = p.float().to(DEV) if mode == "master" else None
    bits = _bits(p)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    ms = p.float().numpy().copy() if mode == "master" else None
    be = backend_for(DEV)
    for step in (1, 2, 3):
        g = (torch.randn(n, generator=gen) * 0.1).float()
        gd = g.to(DEV)
        seed = 40 + step
        be.adam(pd, gd, md, vd, HP["lr"], HP["b1"], HP["b2"], HP["eps"], HP["wd"], 1 - HP["b1"] ** step,
                1 - HP["b2"] ** step, master=master, stochastic=mode == "stochastic", seed=seed)
        O.adam_bf16(bits, g.numpy().copy(), m, v, step=step, moments_bf16=moments == torch.bfloat16, master=ms,
                    stochastic=mode == "stochastic", seed=seed, **HP)
        assert not gd.any()
    assert np.array_equal(_bits(pd), bits)
    assert np.array_equal(md.float().cpu().numpy(), m) and np.array_equal(vd.float().cpu().numpy(), v)
    if mode == "master":
        assert np.array_equal(master.cpu().numpy(), ms)


@pytest.mark.parametrize("master_weights,stochastic", [(False, True), (True, True), (False, False)])
def test_fused_adamw_bf16_parameters(master_weights, stochastic):
    """Two bf16 parameters with fp32 main_grad, two steps: launches use seeds 1, 2, 3, 4 in order
    (the reference increments _seed once per launch), masters live in the optimizer state."""
    gen = torch.Generator().manual_seed(8)
    shapes = [(300, 7), (1001,)]
    params = [torch.nn.Parameter((torch.randn(s, generator=gen) * 0.3).to(torch.bfloat16).to(DEV)) for s in shapes]
    ref = [(_bits(p.reshape(-1)), np.zeros(p.numel(), np.float32), np.zeros(p.numel(), np.float32),
            p.detach().float().reshape(-1).cpu().numpy().copy() if master_weights else None) for p in params]
    opt = FusedAdamW(params, lr=HP["lr"], betas=(HP["b1"], HP["b2"]), eps=HP["eps"], weight_decay=HP["wd"],
                     moments="fp32", master_weights=master_weights, stochastic_rounding=stochastic)
    seed = 0
    for step in (1, 2):
        for p, (bits, m, v, ms) in zip(params, ref):
            g = torch.randn(p.shape, generator=gen).float()
            p.main_grad = g.to(DEV)
            seed += 1
            O.adam_bf16(bits, g.reshape(-1).numpy().copy(), m, v, step=step, master=ms,
                        stochastic=stochastic and not master_weights, seed=seed, **HP)
        opt.step()
    for p, (bits, m, v, ms) in zip(params, ref):
        assert np.array_equal(_bits(p.reshape(-1)), bits)
        st = opt.state[p]
        assert ("master" in st) == master_weights
        if master_weights:
            assert np.array_equal(st["master"].reshape(-1).cpu().numpy(), ms)
