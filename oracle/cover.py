"""TEST INFRASTRUCTURE ONLY: CPU restatement of the Cover-TopK/16 support selection.

Only ``tests/`` may import this module, as the checker of the HIP selection kernel
(granulelayer_amd/csrc/gl_cover.hip); the product package never imports it.  Plain numpy and
Python loops, meant for small envelopes.

The envelope: logical records of C neurons (C a multiple of 16) sharing one record of 64 input
candidates; a record's neurons are cut into row groups of 16 (u = record * C/16 + c // 16), and the
valid neurons of a record are a prefix (nv[u] valid neurons in group u).  Per valid row group:

* ``importance``   a[u, j] = sum over the valid neurons c of u of W[u, c, j]^2 in float64, added in
                   order c = 0..15 (sparse_pooling/experimental/local_supports.py:209-222);
* ``topk``         the k largest a[u, j], ties to the lower candidate position (a stable descending
                   sort), returned as sorted positions (local_supports.py:279-282);
* ``cover_repair`` inside each record every one of the 64 candidates must be kept by at least one
                   valid group: while some candidate j is uncovered, apply the swap (u, d -> j) of
                   smallest energy loss a[u, d] - a[u, j] over every uncovered j, valid group u and
                   retained donor d whose record count is >= 2; ties go to the smallest (j, u) and, for
                   the donor, the smallest d (local_supports.py:294-375).  Records with m valid
                   groups and m k < 64 are infeasible (ValueError).

Parity status: pinned by brute force (every greedy swap is the minimum over an explicit enumeration
of all legal swaps; coverage and degree invariants; exhaustive top-k on tiny inputs) and by vectors
the reference wrote (tests/golden/make_cover_golden.py, tests/test_cover.py).
"""
from __future__ import annotations

import numpy as np

S = 64


def importance(w, nv):
    """a [n16, 64] float64 from w [n16, 16, 64] (fp32 values) and nv [n16] valid neurons per group."""
    w = np.asarray(w, np.float32)
    n16 = w.shape[0]
    a = np.zeros((n16, S), np.float64)
    for u in range(n16):
        acc = np.zeros(S, np.float64)
        for c in range(16):
            x = w[u, c].astype(np.float64) if c < nv[u] else np.zeros(S, np.float64)
            acc = acc + x * x
        a[u] = acc
    return a


def topk(a_row, k):
    """Sorted positions of the k largest values of one row (ties to the lower position)."""
    order = sorted(range(S), key=lambda j: (-a_row[j], j))
    return sorted(order[:k])


def cover_repair(a, env0, nv, gpb, k, trace=False):
    """Repair the supports env0 [n16, k] of records of gpb consecutive groups.  Returns (env [n16, k],
    missing0 [R], swaps [R], loss [R] float64[, per-record list of applied swaps (j, u, d, cost)])."""
    n16 = len(nv)
    R = n16 // gpb
    env = np.array(env0, np.int64).copy()
    missing0 = np.zeros(R, np.int64)
    swaps = np.zeros(R, np.int64)
    loss = np.zeros(R, np.float64)
    log = []
    for r in range(R):
        us = [r * gpb + i for i in range(gpb) if nv[r * gpb + i] > 0]
        rec_log = []
        if not us:
            log.append(rec_log)
            continue
        if len(us) * k < S:
            raise ValueError(f"record {r}: {len(us)} valid groups x k = {k} < {S}")
        keep = {u: set(int(j) for j in env[u]) for u in us}
        count = [sum(j in keep[u] for u in us) for j in range(S)]
        missing0[r] = sum(c == 0 for c in count)
        while any(c == 0 for c in count):
            best = None
            for j in range(S):
                if count[j]:
                    continue
                for u in us:
                    donors = [d for d in sorted(keep[u]) if count[d] >= 2]
                    if not donors:
                        continue
                    d = min(donors, key=lambda dd: (a[u, dd], dd))
                    cost = a[u, d] - a[u, j]
                    if best is None or cost < best[3]:
                        best = (j, u, d, cost)
            if best is None:
                raise AssertionError("an uncovered input without a legal swap")
            j, u, d, cost = best
            keep[u].remove(d)
            keep[u].add(j)
            count[d] -= 1
            count[j] += 1
            swaps[r] += 1
            loss[r] += cost
            rec_log.append(best)
        for u in us:
            env[u] = sorted(keep[u])
        log.append(rec_log)
    out = (env, missing0, swaps, loss)
    return out + (log,) if trace else out


def select(w, nv, gpb, k=16, repair=True):
    """importance -> top-k -> (cover repair) of an envelope w [n16, 16, 64]; padded groups get
    arange(k).  Returns (env [n16, k], importance, missing0, swaps, loss)."""
    a = importance(w, nv)
    env0 = np.array([topk(a[u], k) if nv[u] > 0 else list(range(k)) for u in range(len(nv))], np.int64)
    if not repair:
        R = len(nv) // gpb
        return env0, a, np.zeros(R, np.int64), np.zeros(R, np.int64), np.zeros(R, np.float64)
    env, m0, sw, lo = cover_repair(a, env0, nv, gpb, k)
    return env, a, m0, sw, lo
