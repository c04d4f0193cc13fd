"""Writes randint_triton.npz: Triton's own tl.randint(seed, offset) (triton/language/random.py) for
int64 offsets, run in Triton's CPU interpreter (TRITON_INTERPRET=1), for the stochastic rounding
of FusedAdamW (sparse_pooling/optim.py:59-62 draws tl.randint(seed, offs) with int64 element
offsets).  Triton is a third-party library of the build image (3.6 here; the reference pins 3.3.0,
whose source is not in the image).  Run once in the build container:

    TRITON_INTERPRET=1 python tests/golden/make_randint_golden.py
"""
import os
import sys

import numpy as np

if os.environ.get("TRITON_INTERPRET") != "1":
    sys.exit("run with TRITON_INTERPRET=1 (Triton's CPU interpreter)")

import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402


@triton.jit
def _randint(out, offs_ptr, seed, n, BLOCK: tl.constexpr):
    i = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = i < n
    o = tl.load(offs_ptr + i, mask=m, other=0)
    tl.store(out + i, tl.randint(seed, o), mask=m)


def main():
    offsets = np.array([0, 1, 2, 3, 4, 5, 1000, 65535, 65536, 2**31 - 1, 2**31, 2**32 - 1, 2**32, 2**32 + 5,
                        805_306_367, 2**40 + 17, 2**62 + 3], dtype=np.int64)
    seeds = np.array([1, 2, 7, 12345, 2**31 - 1], dtype=np.int64)
    vals = np.zeros((len(seeds), len(offsets)), dtype=np.uint32)
    offs_t = torch.from_numpy(offsets)
    for si, seed in enumerate(seeds.tolist()):
        out = torch.zeros(len(offsets), dtype=torch.int32)
        _randint[(1,)](out, offs_t, seed, len(offsets), BLOCK=32)
        vals[si] = out.numpy().view(np.uint32)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "randint_triton.npz")
    np.savez(path, seeds=seeds, offsets=offsets, values=vals, triton_version=np.array(triton.__version__))
    print("wrote", path)


if __name__ == "__main__":
    main()
