"""TEST INFRASTRUCTURE ONLY: CPU oracle of the sparse projection -> activation -> pool path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this
module, and only as the checker.  The product package ``granulelayer_amd`` never imports it.

Contents (each restates the reference; file:line citations are relative to the reference root):

* ``forward`` / ``forward_max`` / ``forward_topk`` / ``backward`` / ``backward_topk`` -- float64 C
  restatement (``gl_oracle.c``) of
  ``sparse_pooling/reference/pytorch_reference.py:29-79`` (Mode A) and of the recompute backward
  ``sparse_pooling/kernels/triton_fused.py:364-445`` + ``kernels/ops.py:242-249``.
* ``forward_smooth`` / ``backward_smooth`` -- LogMeanExp, power mean and softmax-weighted pooling
  (``pytorch_reference.py:80-100``; coefficients ``kernels/ops.py:242-262``, dz
  ``kernels/triton_fused.py:364-399``), float64.
* ``adam`` -- fp32 restatement of ``sparse_pooling/optim.py:26-64`` (fp32 parameters).
* ``partition`` -- group partition of ``sparse_pooling/layout.py:68-120``.
* ``xedges`` -- the input-major (transposed) edge list consumed by the HIP dX kernel, in its exact
  bit layout; the order follows the deterministic fixed-owner reduction idea of
  ``sparse_pooling/kernels/cuda/sg_det.cu:1-46`` (every destination summed in a static order).

Parity status (what pins each function; see tests/test_oracle.py):
  forward   pinned: dense-GEMM restatement via torch.matmul, one-hot inputs (closed form),
            mean = sum / n_g, padded-slot masking, hand-computed known answer.
  forward_max pinned: dense-GEMM z with torch.max / torch.argmax (first maximum), hand-built
            ties (smaller slot wins, padded slots never win, relu all-zero pools).
  forward_topk pinned: dense-GEMM z with torch.sort(descending, stable) (the reference's own
            formula, pytorch_reference.py:68-77), hand-built ties and short pools (n_g < k).
  backward  pinned: torch autograd of the dense-GEMM forward, float64 central differences; max
            pooling: autograd of the winner gather (pytorch_reference.py:61-67); top-k mean:
            autograd of the selected-value mean.
  forward_smooth / backward_smooth pinned: torch float64 logsumexp / softmax / pow of the dense z
            and its autograd (tests/test_oracle.py), float64 central differences.
  adam      pinned: torch.optim.Adam / AdamW (library), step-1 closed form.
  partition pinned: invariants of test_sparse_projection.py:14-27 (enumerates range(H)).
  xedges    pinned: brute force per feature on tiny inputs; invariants (permutation of the valid
            edges, per-feature order, segment bookkeeping).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libgl_oracle.so"
_lib = None


def build() -> Path:
    """Compile the C oracle (gcc) into oracle/_build/."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        i, f = ctypes.c_int, ctypes.c_float
        lib.glo_forward_f64.argtypes = [i, i, i, i, i, P, P, P, P, P, i, i, P, P]
        lib.glo_backward_f64.argtypes = [i, i, i, i, i, P, P, P, P, P, i, i, P, P, P, P, ctypes.c_double,
                                         P, P, P, P, P, P]
        lib.glo_adam_f32.argtypes = [ctypes.c_long, P, P, P, P, f, f, f, f, f, f, f, i]
        lib.glo_forward_max_f64.argtypes = [i, i, i, i, i, P, P, P, P, P, i, P, P, P]
        lib.glo_forward_topk_f64.argtypes = [i, i, i, i, i, P, P, P, P, P, i, i, P, P, P]
        lib.glo_backward_topk_f64.argtypes = [i, i, i, i, i, P, P, P, P, P, i, i, P, P, P, P, ctypes.c_double,
                                              P, P, P, P, P, P]
        lib.glo_backward_events_f64.argtypes = [i, i, i, i, i, P, P, P, P, P, i, i, i, P, P, P, P, P, P, P, P]
        d = ctypes.c_double
        lib.glo_forward_smooth_f64.argtypes = [i, i, i, i, i, P, P, P, P, P, i, i, d, P, P, P]
        lib.glo_backward_smooth_f64.argtypes = [i, i, i, i, i, P, P, P, P, P, i, i, d, P, P, P, P, P, P, P]
        u64 = ctypes.c_uint64
        lib.glo_philox4x32.argtypes = [P, P, P]
        lib.glo_randint.argtypes = [u64, u64]
        lib.glo_randint.restype = ctypes.c_uint32
        lib.glo_adam_bf16.argtypes = [ctypes.c_long, P, P, P, P, P, f, f, f, f, f, f, f, i, i, u64]
        for fn in (lib.glo_forward_f64, lib.glo_backward_f64, lib.glo_adam_f32, lib.glo_forward_max_f64,
                   lib.glo_forward_topk_f64, lib.glo_backward_topk_f64, lib.glo_backward_events_f64,
                   lib.glo_forward_smooth_f64, lib.glo_backward_smooth_f64, lib.glo_philox4x32,
                   lib.glo_adam_bf16):
            fn.restype = None
        _lib = lib
    return _lib


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def _shapes(x, idx, counts, S):
    x = np.asarray(x)
    B, D = x.shape
    NS, K = idx.shape
    G = len(counts)
    if NS != G * S:
        raise ValueError(f"idx has {NS} slots, expected G*S = {G * S}")
    return B, D, G, K


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def forward(x, idx, w, bias, counts, S, act="relu", pool="mean", with_mag=False):
    """pre [B, G] float64 (and, with_mag, the error scale ``mag`` [B, G]: scale_g * sum over the
    group of sum_k |x w| + |bias|).  x [B, D] (fp32 values), idx/w [G*S, K], bias [G*S], counts [G]."""
    B, D, G, K = _shapes(x, idx, counts, S)
    x, px = _c(x, np.float32)
    idx, pi = _c(idx, np.int32)
    w, pw = _c(np.asarray(w).reshape(G * S, K), np.float32)
    bias, pb = _c(np.asarray(bias).reshape(G * S), np.float32)
    counts, pc = _c(counts, np.int32)
    pre = np.zeros((B, G), np.float64)
    mag = np.zeros((B, G), np.float64) if with_mag else None
    _load().glo_forward_f64(B, D, G, S, K, px, pi, pw, pb, pc, _ACT[act], _POOL[pool], _p(pre), _p(mag))
    return (pre, mag) if with_mag else pre


def forward_max(x, idx, w, bias, counts, S, act="identity"):
    """Max pooling: (pre [B, G] float64, winner [B, G] int32 pool-local slot, gap [B, G]).  gap is
    the lead of the maximum over the runner-up relative to the rounding scale of z; pairs with a
    gap below ~1e-6 may pick another winner in fp32."""
    B, D, G, K = _shapes(x, idx, counts, S)
    x, px = _c(x, np.float32)
    idx, pi = _c(idx, np.int32)
    w, pw = _c(np.asarray(w).reshape(G * S, K), np.float32)
    bias, pb = _c(np.asarray(bias).reshape(G * S), np.float32)
    counts, pc = _c(counts, np.int32)
    pre = np.zeros((B, G), np.float64)
    win = np.zeros((B, G), np.int32)
    gap = np.zeros((B, G), np.float64)
    _load().glo_forward_max_f64(B, D, G, S, K, px, pi, pw, pb, pc, _ACT[act], _p(pre), _p(win), _p(gap))
    return pre, win, gap


def forward_topk(x, idx, w, bias, counts, S, k, act="identity"):
    """Top-k mean pooling: (pre [B, G] float64, slots [B, G, k] int32 best first, -1 past
    min(n_g, k), gap [B, G]).  gap is the lead of the last selected z over the best unselected one,
    relative to the rounding scale of z; pairs with a gap below ~1e-6 may select another set in fp32."""
    B, D, G, K = _shapes(x, idx, counts, S)
    x, px = _c(x, np.float32)
    idx, pi = _c(idx, np.int32)
    w, pw = _c(np.asarray(w).reshape(G * S, K), np.float32)
    bias, pb = _c(np.asarray(bias).reshape(G * S), np.float32)
    counts, pc = _c(counts, np.int32)
    pre = np.zeros((B, G), np.float64)
    slots = np.zeros((B, G, k), np.int32)
    gap = np.zeros((B, G), np.float64)
    _load().glo_forward_topk_f64(B, D, G, S, K, px, pi, pw, pb, pc, _ACT[act], k, _p(pre), _p(slots), _p(gap))
    return pre, slots, gap


def backward_topk(x, idx, w, bias, counts, S, dy, k, act="identity", with_bounds=False):
    """(dW, db, dX) float64 of top-k mean pooling (the kk selected neurons get dy / kk)."""
    B, D, G, K = _shapes(x, idx, counts, S)
    x, px = _c(x, np.float32)
    idx, pi = _c(idx, np.int32)
    w, pw = _c(np.asarray(w).reshape(G * S, K), np.float32)
    bias, pb = _c(np.asarray(bias).reshape(G * S), np.float32)
    counts, pc = _c(counts, np.int32)
    dy, pdy = _c(dy, np.float32)
    shapes = ((G * S, K), (G * S,), (B, D))
    dW, db, dX = (np.zeros(s, np.float64) for s in shapes)
    mag = tuple(np.zeros(s, np.float64) for s in shapes) if with_bounds else (None,) * 3
    unc = tuple(np.zeros(s, np.float64) for s in shapes) if with_bounds else (None,) * 3
    _load().glo_backward_topk_f64(B, D, G, S, K, px, pi, pw, pb, pc, _ACT[act], k, pdy, _p(dW), _p(db), _p(dX),
                                  AMBIGUOUS_Z, *map(_p, mag), *map(_p, unc))
    if with_bounds:
        return dW, db, dX, {"mag": mag, "unc": unc}
    return dW, db, dX


def backward_events(x, idx, w, bias, counts, S, dy, slots, act="identity", topk=False):
    """(dW, db, dX, (magW, magb, magX)) float64 of a given selection: slots [B, G] (max pooling) or
    [B, G, k] (top-k mean, coef dy / min(n_g, k)); -1 = none.  With the pooling's own selection it
    equals backward(pool="max") / backward_topk."""
    B, D, G, K = _shapes(x, idx, counts, S)
    x, px = _c(x, np.float32)
    idx, pi = _c(idx, np.int32)
    w, pw = _c(np.asarray(w).reshape(G * S, K), np.float32)
    bias, pb = _c(np.asarray(bias).reshape(G * S), np.float32)
    counts, pc = _c(counts, np.int32)
    dy, pdy = _c(dy, np.float32)
    slots = np.asarray(slots, np.int32).reshape(B, G, -1)
    kpe = slots.shape[2]
    slots, ps = _c(slots, np.int32)
    shapes = ((G * S, K), (G * S,), (B, D))
    dW, db, dX = (np.zeros(s, np.float64) for s in shapes)
    mag = tuple(np.zeros(s, np.float64) for s in shapes)
    _load().glo_backward_events_f64(B, D, G, S, K, px, pi, pw, pb, pc, _ACT[act], int(topk), kpe, ps, pdy, _p(dW),
                                    _p(db), _p(dX), *map(_p, mag))
    return dW, db, dX, mag


# relu masks decided within this relative distance of z = 0 may differ in fp32 (z is a sum of
# K + 1 terms: its fp32 rounding error stays below (K + 1) * 2^-24 * sum|terms|)
AMBIGUOUS_Z = 1e-6


def backward(x, idx, w, bias, counts, S, dy, act="relu", pool="mean", with_bounds=False):
    """(dW [G*S, K], db [G*S], dX [B, D]) float64 for upstream gradient dy [B, G].  with_bounds
    also returns {"mag": (magW, magb, magX), "unc": (uncW, uncb, uncX)} (see gl_oracle.c)."""
    B, D, G, K = _shapes(x, idx, counts, S)
    x, px = _c(x, np.float32)
    idx, pi = _c(idx, np.int32)
    w, pw = _c(np.asarray(w).reshape(G * S, K), np.float32)
    bias, pb = _c(np.asarray(bias).reshape(G * S), np.float32)
    counts, pc = _c(counts, np.int32)
    dy, pdy = _c(dy, np.float32)
    shapes = ((G * S, K), (G * S,), (B, D))
    dW, db, dX = (np.zeros(s, np.float64) for s in shapes)
    mag = tuple(np.zeros(s, np.float64) for s in shapes) if with_bounds else (None,) * 3
    unc = tuple(np.zeros(s, np.float64) for s in shapes) if with_bounds else (None,) * 3
    _load().glo_backward_f64(B, D, G, S, K, px, pi, pw, pb, pc, _ACT[act], _POOL[pool], pdy, _p(dW), _p(db), _p(dX),
                             AMBIGUOUS_Z, *map(_p, mag), *map(_p, unc))
    if with_bounds:
        return dW, db, dX, {"mag": mag, "unc": unc}
    return dW, db, dX


# pool codes of the smooth operators (gl_oracle.c); param: temperature, p or beta
SMOOTH = {"logmeanexp": 4, "power_mean": 5, "softmax_weighted": 6}


def _operands(x, idx, w, bias, counts, S):
    B, D, G, K = _shapes(x, idx, counts, S)
    x, px = _c(x, np.float32)
    idx, pi = _c(idx, np.int32)
    w, pw = _c(np.asarray(w).reshape(G * S, K), np.float32)
    bias, pb = _c(np.asarray(bias).reshape(G * S), np.float32)
    counts, pc = _c(counts, np.int32)
    return (B, D, G, K), (x, idx, w, bias, counts), (px, pi, pw, pb, pc)


def forward_smooth(x, idx, w, bias, counts, S, pool, param, act="identity"):
    """LogMeanExp (param = temperature), power mean (param = p, relu activations) or softmax-weighted
    (param = beta) pooling: (pre [B, G], lse [B, G] the log2-normaliser (0 for power), mag [B, G] the
    scale of an fp32 evaluation's error), float64 (pytorch_reference.py:80-100)."""
    (B, D, G, K), keep, ptrs = _operands(x, idx, w, bias, counts, S)
    pre, lse, mag = (np.zeros((B, G), np.float64) for _ in range(3))
    _load().glo_forward_smooth_f64(B, D, G, S, K, *ptrs, _ACT[act], SMOOTH[pool], float(param), _p(pre), _p(lse),
                                   _p(mag))
    return pre, lse, mag


def backward_smooth(x, idx, w, bias, counts, S, dy, pool, param, act="identity"):
    """(dW, db, dX, (magW, magb, magX)) float64 of the smooth pooling operators for upstream dy [B, G]
    (kernels/ops.py:242-262 coefficients, triton_fused.py:364-399 dz)."""
    (B, D, G, K), keep, ptrs = _operands(x, idx, w, bias, counts, S)
    dy, pdy = _c(dy, np.float32)
    shapes = ((G * S, K), (G * S,), (B, D))
    dW, db, dX = (np.zeros(s, np.float64) for s in shapes)
    mag = tuple(np.zeros(s, np.float64) for s in shapes)
    _load().glo_backward_smooth_f64(B, D, G, S, K, *ptrs, _ACT[act], SMOOTH[pool], float(param), pdy, _p(dW), _p(db),
                                    _p(dX), *map(_p, mag))
    return dW, db, dX, mag


def adam(p, g, m, v, lr, b1, b2, eps, wd, step, moments_bf16=False):
    """In-place fp32 AdamW step (numpy float32 arrays); bias corrections 1 - beta**step (float64,
    then fp32, as the reference passes Python floats to the kernel: optim.py:119-123)."""
    for a in (p, g, m, v):
        if a.dtype != np.float32 or not a.flags["C_CONTIGUOUS"]:
            raise TypeError("adam expects contiguous float32 arrays")
    bc1, bc2 = 1.0 - b1 ** step, 1.0 - b2 ** step
    P = ctypes.c_void_p
    _load().glo_adam_f32(p.size, p.ctypes.data_as(P), g.ctypes.data_as(P), m.ctypes.data_as(P),
                         v.ctypes.data_as(P), lr, b1, b2, eps, wd, bc1, bc2, int(moments_bf16))


def philox4x32(ctr, key):
    """Philox-4x32-10 output (4 uint32) of counter ctr (4 uint32) and key key (2 uint32)."""
    c = np.ascontiguousarray(ctr, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    out = np.zeros(4, np.uint32)
    P = ctypes.c_void_p
    _load().glo_philox4x32(c.ctypes.data_as(P), k.ctypes.data_as(P), out.ctypes.data_as(P))
    return out


def randint(seed: int, offset: int) -> int:
    """Triton's tl.randint(seed, offset) for a 64-bit offset (Triton 3.6 randint4x)."""
    return int(_load().glo_randint(seed, offset))


def adam_bf16(p_bits, g, m, v, lr, b1, b2, eps, wd, step, moments_bf16=False, master=None, stochastic=True, seed=0):
    """In-place AdamW step of bf16 parameters (p_bits: numpy uint16 bf16 patterns; g, m, v and the
    optional fp32 master copy: float32), the HAS_MASTER / STOCH branches of optim.py:26-64."""
    if p_bits.dtype != np.uint16 or not p_bits.flags["C_CONTIGUOUS"]:
        raise TypeError("adam_bf16 expects contiguous uint16 parameter bits")
    for a in (g, m, v) + (() if master is None else (master,)):
        if a.dtype != np.float32 or not a.flags["C_CONTIGUOUS"]:
            raise TypeError("adam_bf16 expects contiguous float32 g / m / v / master")
    bc1, bc2 = 1.0 - b1 ** step, 1.0 - b2 ** step
    P = ctypes.c_void_p
    _load().glo_adam_bf16(p_bits.size, p_bits.ctypes.data_as(P), None if master is None else master.ctypes.data_as(P),
                          g.ctypes.data_as(P), m.ctypes.data_as(P), v.ctypes.data_as(P), lr, b1, b2, eps, wd, bc1,
                          bc2, int(moments_bf16), int(stochastic), seed)


_ACT = {"identity": 0, "relu": 1, "gelu": 2}
_POOL = {"mean": 0, "sum": 1, "max": 2}


def partition(H: int, G: int, block: int = 8):
    """(counts [G], offsets [G], S) of layout.py:68-120: n_g = H//G + (g < H%G), group offset
    g*(H//G) + min(g, H%G), blocks of ``block`` slots padded to a multiple of 4 blocks."""
    base, rem = divmod(H, G)
    g = np.arange(G, dtype=np.int64)
    counts = base + (g < rem).astype(np.int64)
    offsets = g * base + np.minimum(g, rem)
    max_group = base + (1 if rem else 0)
    nb = -(-max_group // block)
    nb = (nb + 3) // 4 * 4
    return counts.astype(np.int32), offsets, nb * block


# ----------------------------------------------------------------------------------------------
# transposed (input-major) edge list of the HIP dX kernel
# ----------------------------------------------------------------------------------------------
# record = (n_local * K + k) * 4 | f_local << 16 | newf << 31, where n_local is the slot inside
# the unit and newf marks an edge whose feature differs from the previous edge of its segment
REC_F_SHIFT, REC_NEWF = 16, 1 << 31


def xedges(idx, counts, S, D, Fw, US):
    """Input-major edge structure of the dX kernel, as numpy arrays (bit-exact specification).

    Valid edges (slot s < counts[g]) are ordered by the key
        (F = d // Fw, unit u, f_local = d % Fw, eid = n*K + k)
    where unit u = g * P + s // US (P = ceil(S / US) pieces per group) and n = g*S + s.
    Returns dict:
      rec       uint32 [E]   (n_local * K + k) * 4 | f_local << 16 | newf << 31   (n_local = s % US;
                             newf: same segment as the previous edge, different feature)
      seg_ptr   int64 [FR+1] segment range of feature range F
      seg_unit  int32 [nseg] unit of each (F, u) segment with at least one edge, ascending in u
      seg_begin int64 [nseg+1] first edge of each segment (+ total E)
    """
    idx = np.asarray(idx, np.int64)
    NS, K = idx.shape
    G = len(counts)
    P = -(-S // US)
    FR = -(-D // Fw)
    n = np.arange(NS, dtype=np.int64)
    g = n // S
    s = n % S
    valid = s < np.asarray(counts, np.int64)[g]
    nn = np.repeat(n[valid], K)
    kk = np.tile(np.arange(K, dtype=np.int64), int(valid.sum()))
    d = idx[valid].reshape(-1)
    u = (nn // S) * P + (nn % S) // US
    eid = nn * K + kk
    F = d // Fw
    fl = d % Fw
    order = np.lexsort((eid, fl, u, F))
    Fo, uo, flo = F[order], u[order], fl[order]
    key = Fo * (G * P) + uo
    newf = np.zeros(len(key), bool)
    if len(key) > 1:
        newf[1:] = (key[1:] == key[:-1]) & (flo[1:] != flo[:-1])
    el = ((nn % S) % US) * K + kk
    rec = (el[order] * 4) | (flo << REC_F_SHIFT) | (newf.astype(np.int64) << 31)
    if len(key):
        starts = np.concatenate([[0], np.nonzero(np.diff(key))[0] + 1])
    else:
        starts = np.zeros(0, np.int64)
    seg_F = Fo[starts] if len(key) else np.zeros(0, np.int64)
    seg_ptr = np.searchsorted(seg_F, np.arange(FR + 1), side="left").astype(np.int64)
    seg_begin = np.concatenate([starts, [len(key)]]).astype(np.int64)
    return dict(rec=rec.astype(np.uint32), seg_ptr=seg_ptr, seg_unit=uo[starts].astype(np.int32),
                seg_begin=seg_begin, FR=FR, P=P, U=G * P)
