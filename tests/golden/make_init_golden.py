"""Writes tests/golden/init_reference.npz: the reference's seeded parameter initialisation
(sparse_pooling/layout.py:191-251, init_parameters with _sample_distinct and zero_padding_) for a
ragged Mode-A layout (padded slots in every group) at two seeds, and with a bias std.

The product restates those steps (granulelayer_amd/layout.py) so that SparsePoolingLayer(seed=s)
yields the reference's parameters bit for bit; tests/test_host.py checks it against this file.
The reference only runs here, in the build container, to write the vectors: the fixture holds data
(inputs and outputs), never reference code.  Usage (repository root):

    python tests/golden/make_init_golden.py /root/reference
"""
import sys
from pathlib import Path

import numpy as np
import torch

CASES = [
    # name, input_dim, hidden_dim, groups, seed, dtype, bias_std, chunk_records
    ("s0", 300, 2000, 7, 0, torch.float32, 0.0, 1 << 22),
    ("s7", 1024, 2345, 13, 7, torch.float32, 0.25, 1 << 22),
    ("s3_chunked", 64, 3001, 5, 3, torch.float32, 0.0, 500),
    ("s5_bf16", 200, 999, 4, 5, torch.bfloat16, 0.1, 1 << 22),
]


def main(ref_root: str):
    sys.path.insert(0, ref_root)
    from sparse_pooling.layout import SparseLayout, init_parameters

    out = {}
    for name, D, H, G, seed, dtype, bias_std, chunk in CASES:
        L = SparseLayout(D, H, G, 8, 8, False)
        idx, w, b = init_parameters(L, "cpu", dtype=dtype, seed=seed, bias_std=bias_std, chunk_records=chunk)
        out[f"{name}/shape"] = np.array([D, H, G, seed, chunk], np.int64)
        out[f"{name}/bias_std"] = np.array(bias_std, np.float64)
        out[f"{name}/dtype"] = np.array(str(dtype).replace("torch.", ""))
        out[f"{name}/idx"] = idx.numpy()  # int16, as the reference stores Mode-A indices
        out[f"{name}/w"] = w.float().numpy()  # bf16 values widened exactly
        out[f"{name}/b"] = b.float().numpy()
    path = Path(__file__).resolve().parent / "init_reference.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
