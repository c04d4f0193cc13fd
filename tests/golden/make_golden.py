"""Write tests/golden/golden_small.npz: small known-answer vectors for the Mode-A path.

The reference ships no numeric golden vectors for this path, so these are computed with torch
library routines only, independently of the C oracle:
  * the forward as a dense matrix product: W scattered into a dense [G*S, D] matrix (zero rows
    for padded slots), z = X @ Wd^T + bias, ReLU, masked mean or sum over each pool
    (sparse_pooling/reference/pytorch_reference.py:29-79 semantics), in float64;
  * dX, dW, db by torch autograd of that dense forward (float64), for an upstream gradient dY;
  * three AdamW steps by torch.optim.AdamW on fp32 tensors (sparse_pooling/optim.py:26-64
    semantics; the reference's own Adam test compares against the same library,
    tests/test_optim.py:11-28).

Run from the repository root: ``python tests/golden/make_golden.py``.  Output is deterministic
(numpy seed 20251201 for inputs; torch only does arithmetic).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "golden_small.npz"

CASES = [
    # name, B, D, G, S, K, pool, counts
    ("mean_k8", 7, 48, 5, 32, 8, "mean", [32, 31, 20, 25, 1]),
    ("sum_k8", 9, 40, 4, 32, 8, "sum", [32, 17, 29, 3]),
    ("sum_k16", 5, 64, 3, 32, 16, "sum", [30, 32, 9]),
]


def _case(rng, B, D, G, S, K, pool, counts):
    counts = np.asarray(counts, np.int32)
    NS = G * S
    idx = np.zeros((NS, K), np.int32)
    for n in range(NS):
        idx[n] = np.sort(rng.choice(D, size=K, replace=False))
    w = rng.normal(0.0, 1.0 / np.sqrt(K), (NS, K)).astype(np.float32)
    b = rng.normal(0.0, 0.2, NS).astype(np.float32)
    valid = (np.arange(S)[None, :] < counts[:, None]).reshape(-1)
    w[~valid] = 0.0
    b[~valid] = 0.0
    idx[~valid] = 0
    x = rng.normal(0.0, 1.0, (B, D)).astype(np.float32)
    dy = rng.normal(0.0, 1.0, (B, G)).astype(np.float32)

    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    dense = torch.zeros(NS, D, dtype=torch.float64)
    rows = torch.arange(NS).repeat_interleave(K)
    dense = dense.index_put((rows, torch.tensor(idx.reshape(-1), dtype=torch.long)), wt.reshape(-1),
                            accumulate=True)
    z = xt @ dense.t() + bt
    a = torch.relu(z) * torch.tensor(valid, dtype=torch.float64)
    s = a.reshape(B, G, S).sum(-1)
    pre = s / torch.tensor(counts, dtype=torch.float64) if pool == "mean" else s
    pre.backward(torch.tensor(dy, dtype=torch.float64))
    return dict(x=x, idx=idx, w=w, b=b, counts=counts, dy=dy, pre=pre.detach().numpy(),
                dX=xt.grad.numpy(), dW=wt.grad.numpy(), db=bt.grad.numpy(),
                shape=np.array([B, D, G, S, K, 0 if pool == "mean" else 1], np.int64))


def _adam(rng):
    n = 1000
    p0 = rng.normal(0.0, 1.0, n).astype(np.float32)
    grads = rng.normal(0.0, 1.0, (3, n)).astype(np.float32)
    p = torch.tensor(p0, requires_grad=True)
    opt = torch.optim.AdamW([p], lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
    for t in range(3):
        p.grad = torch.tensor(grads[t])
        opt.step()
    st = opt.state[p]
    return dict(p0=p0, grads=grads, p=p.detach().numpy(), m=st["exp_avg"].numpy(), v=st["exp_avg_sq"].numpy(),
                hyper=np.array([1e-2, 0.9, 0.999, 1e-8, 0.1], np.float64))


def main():
    rng = np.random.default_rng(20251201)
    out = {}
    for name, B, D, G, S, K, pool, counts in CASES:
        for k, v in _case(rng, B, D, G, S, K, pool, counts).items():
            out[f"{name}/{k}"] = v
    for k, v in _adam(rng).items():
        out[f"adam/{k}"] = v
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
