"""FusedAdamW with bf16 parameters (sparse_pooling/optim.py:5-9, 26-64), CPU side: the oracle's
Philox-4x32-10 against the Random123 known-answer vectors and against Triton's own tl.randint
(tests/golden/randint_triton.npz), and the oracle's three bf16 modes against independent routes:
nearest-even and master weights through the fp32 oracle (pinned against torch.optim.AdamW in
test_oracle.py) and torch's own float32 -> bfloat16 cast; stochastic rounding by its defining
properties (one of the two bf16 neighbours, unbiased)."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "randint_triton.npz")

# Random123 (Salmon et al., SC'11) known-answer vectors of philox4x32-10: counter, key -> output
PHILOX_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX_KAT)
def test_philox_known_answers(ctr, key, want):
    assert tuple(int(x) for x in O.philox4x32(ctr, key)) == want


def test_randint_matches_triton():
    z = np.load(GOLDEN)
    for si, seed in enumerate(z["seeds"].tolist()):
        got = [O.randint(seed, o) for o in z["offsets"].tolist()]
        assert got == z["values"][si].tolist(), f"seed {seed}"


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def _from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(b.view(np.int16).copy()).view(torch.bfloat16)


def _state(n, seed, moments_bf16):
    g = torch.Generator().manual_seed(seed)
    p = (torch.randn(n, generator=g) * 0.3).to(torch.bfloat16)
    grad = (torch.randn(n, generator=g) * 0.1).numpy().astype(np.float32)
    m = (torch.randn(n, generator=g) * 0.01).numpy().astype(np.float32)
    v = (torch.rand(n, generator=g) * 1e-3).numpy().astype(np.float32)
    if moments_bf16:
        m = torch.from_numpy(m).to(torch.bfloat16).float().numpy()
        v = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    return p, grad, m, v


HP = dict(lr=1e-2, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)


@pytest.mark.parametrize("moments_bf16", [False, True])
def test_nearest_even_is_the_fp32_update_cast_to_bf16(moments_bf16):
    p, g, m, v = _state(1003, 1, moments_bf16)
    bits = _bf16_bits(p)
    g2, m2, v2 = g.copy(), m.copy(), v.copy()
    O.adam_bf16(bits, g2, m2, v2, step=3, moments_bf16=moments_bf16, stochastic=False, **HP)
    p32 = p.float().numpy().copy()
    g3, m3, v3 = g.copy(), m.copy(), v.copy()
    O.adam(p32, g3, m3, v3, step=3, moments_bf16=moments_bf16, **HP)
    want = _bf16_bits(torch.from_numpy(p32).to(torch.bfloat16))
    assert np.array_equal(bits, want)
    assert np.array_equal(m2, m3) and np.array_equal(v2, v3) and not g2.any()


def test_master_weights_run_the_fp32_update_and_round_it():
    p, g, m, v = _state(777, 2, False)
    master = p.float().numpy().copy()
    master[::3] += 1e-4  # the master carries bits the bf16 parameter does not
    bits = _bf16_bits(p)
    ms, g2, m2, v2 = master.copy(), g.copy(), m.copy(), v.copy()
    O.adam_bf16(bits, g2, m2, v2, step=1, master=ms, **HP)
    p32, g3, m3, v3 = master.copy(), g.copy(), m.copy(), v.copy()
    O.adam(p32, g3, m3, v3, step=1, **HP)
    assert np.array_equal(ms, p32)
    assert np.array_equal(bits, _bf16_bits(torch.from_numpy(p32).to(torch.bfloat16)))


def test_stochastic_rounding_picks_a_neighbour_and_is_unbiased():
    """Every result is the bf16 value below or above the fp32 update; over many seeds the mean of
    the rounded values is the fp32 update (the noise is uniform below the cut)."""
    n, trials = 64, 2000
    p, g, m, v = _state(n, 3, False)
    p32 = p.float().numpy().copy()
    O.adam(p32, g.copy(), m.copy(), v.copy(), step=1, **HP)
    u = p32.view(np.uint32)
    lo = (u & 0xFFFF0000).view(np.float32).astype(np.float64)
    hi = ((u & 0xFFFF0000) + 0x10000).view(np.float32).astype(np.float64)
    acc = np.zeros(n)
    for seed in range(1, trials + 1):
        bits = _bf16_bits(p)
        O.adam_bf16(bits, g.copy(), m.copy(), v.copy(), step=1, stochastic=True, seed=seed, **HP)
        got = _from_bits(bits).double().numpy()
        assert np.all((got == lo) | (got == hi))
        acc += got
    mean = acc / trials
    frac = (u & 0xFFFF).astype(np.float64) / 65536.0
    sd = np.abs(hi - lo) * np.sqrt(frac * (1 - frac) / trials)  # (hi is the larger magnitude)
    assert np.all(np.abs(mean - p32.astype(np.float64)) <= 5 * sd + 1e-12)
    # elements and seeds draw different noise
    a, b = _bf16_bits(p), _bf16_bits(p)
    O.adam_bf16(a, g.copy(), m.copy(), v.copy(), step=1, stochastic=True, seed=11, **HP)
    O.adam_bf16(b, g.copy(), m.copy(), v.copy(), step=1, stochastic=True, seed=12, **HP)
    assert not np.array_equal(a, b)
