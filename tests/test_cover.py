"""The Cover-TopK/16 support-selection oracle (oracle/cover.py) on the CPU: against vectors the
reference wrote (tests/golden/make_cover_golden.py: feature_importance, topk_select, cover_repair of
sparse_pooling/experimental/local_supports.py), and against brute force -- every greedy swap is the
first of an explicit enumeration of all legal swaps ordered by (energy loss, j, u, donor order),
coverage >= 1 and degree k hold after the repair, and top-k equals numpy's stable argsort."""
from pathlib import Path

import numpy as np
import pytest

from oracle import cover as C

GOLDEN = Path(__file__).resolve().parent / "golden" / "cover_reference.npz"


def _cases():
    with np.load(GOLDEN) as z:
        d = {k: z[k] for k in z.files}
    names = sorted({k.split("/")[0] for k in d})
    return [(n, {k.split("/", 1)[1]: v for k, v in d.items() if k.startswith(n + "/")}) for n in names]


def _envelope(case):
    H, G, Cb, seed = (int(v) for v in case["shape"])
    w = case["w_int"].astype(np.float32) / 4096  # [G, NB, C, 64]
    return w.reshape(-1, 16, 64), case["nv"], Cb // 16


@pytest.mark.parametrize("name,case", _cases(), ids=lambda c: c if isinstance(c, str) else "")
def test_oracle_matches_reference_vectors(name, case):
    w, nv, gpb = _envelope(case)
    env, a, m0, sw, lo = C.select(w, nv, gpb, 16, repair=True)
    assert np.array_equal(a, case["importance"]), "importance differs from the reference's float64 sums"
    uv = case["valid_groups"]
    env0 = np.array([C.topk(a[u], 16) for u in uv])
    assert np.array_equal(env0, case["env_topk"]), "top-16 differs"
    assert np.array_equal(env[uv], case["env_cover"]), "repaired supports differ"
    rec_valid = np.array([nv[r * gpb:(r + 1) * gpb].sum() > 0 for r in range(len(nv) // gpb)])
    assert np.array_equal(m0[rec_valid], case["missing0"])
    assert np.array_equal(sw[rec_valid], case["swaps"])
    assert np.array_equal(lo[rec_valid], case["loss"]), "energy loss differs (float64 sums in swap order)"


def test_golden_cases_exercise_repairs_ties_and_partial_groups():
    tot_swaps, partial, ties = 0, 0, 0
    for _, case in _cases():
        tot_swaps += int(case["swaps"].sum())
        partial += int(((case["nv"] > 0) & (case["nv"] < 16)).sum())
        a = case["importance"][case["valid_groups"]]
        ties += int(sum(len(r) - len(np.unique(r)) for r in a))
    assert tot_swaps > 100 and partial >= 4 and ties > 1000


def _random_envelope(seed, R, gpb, quant=None):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((R * gpb, 16, 64)).astype(np.float32)
    if quant:
        w = np.round(w * quant).astype(np.float32) / quant
    nv = np.full(R * gpb, 16, np.int64)
    nv[-1] = 5  # a partial group in the last record
    return w, nv


@pytest.mark.parametrize("seed,gpb,quant", [(0, 4, None), (1, 4, 1), (2, 8, 2), (3, 16, None)])
def test_every_greedy_swap_is_the_minimum_of_all_legal_swaps(seed, gpb, quant):
    w, nv = _random_envelope(seed, 6, gpb, quant)
    a = C.importance(w, nv)
    env0 = np.array([C.topk(a[u], 16) for u in range(len(nv))])
    env, m0, sw, lo, log = C.cover_repair(a, env0, nv, gpb, 16, trace=True)
    for r in range(len(nv) // gpb):
        us = [r * gpb + i for i in range(gpb) if nv[r * gpb + i] > 0]
        keep = {u: set(env0[u].tolist()) for u in us}
        total = 0.0
        for (j, u, d, cost) in log[r]:
            count = [sum(x in keep[v] for v in us) for x in range(64)]
            legal = [(a[v, dd] - a[v, jj], jj, v, a[v, dd], dd)
                     for jj in range(64) if count[jj] == 0
                     for v in us for dd in keep[v] if count[dd] >= 2]
            first = min(legal)
            assert (first[1], first[2], first[4]) == (j, u, d), f"record {r}: applied {(j, u, d)}, minimum {first}"
            keep[u].remove(d)
            keep[u].add(j)
            total += cost
        count = [sum(x in keep[v] for v in us) for x in range(64)]
        assert min(count) >= 1 and all(len(keep[v]) == 16 for v in us)
        assert sw[r] == m0[r] == len(log[r]) and lo[r] == total
        for v in us:
            assert env[v].tolist() == sorted(keep[v])


def test_topk_equals_stable_argsort():
    rng = np.random.default_rng(5)
    for _ in range(200):
        row = rng.integers(0, 4, 64).astype(np.float64)  # heavy ties
        k = int(rng.integers(1, 64))
        want = sorted(np.argsort(-row, kind="stable")[:k].tolist())
        assert C.topk(row, k) == want


def test_infeasible_records_are_refused():
    w, nv = _random_envelope(7, 2, 4)
    nv[4:] = [16, 16, 16, 0]  # the second record has 3 valid groups: 3 x 16 < 64
    a = C.importance(w, nv)
    env0 = np.array([C.topk(a[u], 16) for u in range(len(nv))])
    with pytest.raises(ValueError, match="valid groups"):
        C.cover_repair(a, env0, nv, 4, 16)
