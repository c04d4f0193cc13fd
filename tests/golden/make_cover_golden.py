"""Writes tests/golden/cover_reference.npz: the reference's Cover-TopK support selection on small
envelopes -- feature_importance, topk_select and cover_repair of
sparse_pooling/experimental/local_supports.py:209-222, 279-282, 294-375 on envelope weights laid out
as experimental/kgen_layout.KLayout(D, H, G, 64, C) -- for tests/test_cover.py.

The reference runs only here, in the build container, to produce the vectors; the fixture holds
data (inputs and outputs), never reference code.  Usage (repository root):

    python tests/golden/make_cover_golden.py /root/reference
"""
import sys
from pathlib import Path

import numpy as np
import torch

CASES = [
    # name, hidden, groups, C, seed, integer weight range (coarse values: many importance ties)
    ("c256", 1200, 3, 256, 0, 30000),
    ("c256_ties", 900, 2, 256, 1, 3),
    ("c64", 768, 4, 64, 2, 30000),
    ("c128_ties", 1000, 3, 128, 3, 2),
]


def main(ref_root: str):
    sys.path.insert(0, ref_root)
    from sparse_pooling.experimental import local_supports as LS
    from sparse_pooling.experimental.kgen_layout import KLayout

    out = {}
    for name, H, G, C, seed, quant in CASES:
        L = KLayout(4096, H, G, 64, C)
        gen = torch.Generator().manual_seed(seed)
        # weights i / 4096 for integers |i| <= quant: exact in fp32 and stored as int16
        wi = torch.randint(-quant, quant + 1, L.weight_shape, generator=gen, dtype=torch.int64).to(torch.int16)
        valid = L.valid_mask("cpu")
        wi = wi * valid[..., None]
        w = wi.to(torch.float32) / 4096
        a = LS.feature_importance(w, L)  # [n16, 64] float64
        nv = valid.reshape(-1, 16).sum(1)
        uv = torch.nonzero(nv > 0).squeeze(1)
        env0 = LS.topk_select(a[uv], 16)
        gpb = C // 16
        blk = uv // gpb
        blk_valid = torch.zeros(L.groups * L.blocks_per_group, dtype=torch.bool)
        blk_valid[blk] = True
        rec = (torch.cumsum(blk_valid.to(torch.int64), 0) - 1)[blk]
        rank = uv % gpb
        rep = LS.cover_repair(a[uv], env0, rec, rank, 16, gpb)
        out[f"{name}/shape"] = np.array([H, G, C, seed], np.int64)
        out[f"{name}/w_int"] = wi.numpy().astype(np.int16)  # w = w_int / 4096
        out[f"{name}/nv"] = nv.numpy().astype(np.int32)
        out[f"{name}/importance"] = a.numpy()
        out[f"{name}/valid_groups"] = uv.numpy()
        out[f"{name}/env_topk"] = env0.numpy().astype(np.int32)
        out[f"{name}/env_cover"] = rep["env"].numpy().astype(np.int32)
        out[f"{name}/missing0"] = rep["missing0"].numpy()
        out[f"{name}/swaps"] = rep["swaps"].numpy()
        out[f"{name}/loss"] = rep["loss"].numpy()
        print(name, "records", len(rep["swaps"]), "swaps", int(rep["swaps"].sum()))
    path = Path(__file__).resolve().parent / "cover_reference.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
