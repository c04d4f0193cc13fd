"""The CPU oracle against the stored known-answer vectors of tests/golden/ (computed with torch
library routines by tests/golden/make_golden.py: a dense-matrix forward, torch autograd, and
torch.optim.AdamW), so the oracle is pinned by something other than itself."""
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden" / "golden_small.npz"
CASES = ["mean_k8", "sum_k8", "sum_k16"]


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN) as d:  # allow_pickle stays False
        return {k: d[k] for k in d.files}


def case(g, name):
    return {k.split("/", 1)[1]: v for k, v in g.items() if k.startswith(name + "/")}


@pytest.mark.parametrize("name", CASES)
def test_oracle_forward_backward_match_golden(golden, oracle, name):
    c = case(golden, name)
    B, D, G, S, K, pool = (int(v) for v in c["shape"])
    pool = "mean" if pool == 0 else "sum"
    pre = oracle.forward(c["x"], c["idx"], c["w"], c["b"], c["counts"], S, "relu", pool)
    np.testing.assert_allclose(pre, c["pre"], rtol=1e-12, atol=1e-12)
    dW, db, dX = oracle.backward(c["x"], c["idx"], c["w"], c["b"], c["counts"], S, c["dy"], "relu", pool)
    np.testing.assert_allclose(dX, c["dX"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dW, c["dW"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(db, c["db"], rtol=1e-12, atol=1e-12)


def test_golden_cases_cover_padding_and_both_pools(golden):
    for name in CASES:
        c = case(golden, name)
        B, D, G, S, K, pool = (int(v) for v in c["shape"])
        assert c["counts"].min() < S, "every case has padded slots"
        pad = (np.arange(S)[None, :] >= c["counts"][:, None]).reshape(-1)
        assert np.all(c["dW"][pad] == 0) and np.all(c["db"][pad] == 0)
    assert {int(case(golden, n)["shape"][5]) for n in CASES} == {0, 1}
    assert {int(case(golden, n)["shape"][4]) for n in CASES} == {8, 16}


def test_oracle_adam_matches_golden_adamw(golden, oracle):
    a = case(golden, "adam")
    lr, b1, b2, eps, wd = (float(v) for v in a["hyper"])
    p = a["p0"].copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for t in range(3):
        oracle.adam(p, a["grads"][t].copy(), m, v, lr, b1, b2, eps, wd, t + 1)
    # the reference (and the oracle) form 1 - beta in fp32 (fl(1 - fl(0.999)) is 1.3e-5 away from
    # torch's 0.001), so v differs at that relative level and p by well under lr * 1e-4
    np.testing.assert_allclose(m, a["m"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(v, a["v"], rtol=2e-5, atol=1e-9)
    np.testing.assert_allclose(p, a["p"], rtol=0, atol=3 * lr * 1e-4)
