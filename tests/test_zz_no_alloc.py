"""gl_fwd_static, the forward that allocates nothing (its token tiles and partial results live in
the library's static device scratch): through the C ABI, its output equals gl_fwd's bit for bit,
on two calls in a row, the second with a smaller input; a layer whose one-tile partials exceed the
scratch is refused before any device work."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import gpu_available

from granulelayer_amd import LevelSpec, PhysicalPlan
from granulelayer_amd import _native as N
from granulelayer_amd.autograd import Level1Runtime
from granulelayer_amd.backend import HipBackend, _ptr, _stream

DEV = "cuda"


def _args(rt, x, w, b, pre, winner=None, k=0, pool="sum"):
    L = rt.layout
    be = HipBackend.get()
    lo, width = be.windows(rt)
    return N.GlFwdArgs(X=_ptr(x), sxb=x.stride(0), x_dtype=N.GL_DTYPE_F32, B=x.shape[0], D=L.input_dim, G=L.groups,
                       S=L.slots_per_group, K=L.fan_in, act=N.GL_ACT["relu"], pool=N.GL_POOL[pool], topk=k,
                       idx=_ptr(rt.idx), W=_ptr(w), bias=_ptr(b), counts=_ptr(rt.counts_i32),
                       sched=_ptr(be.schedule(rt)), win=_ptr(lo), win_width=width, pre=_ptr(pre), winner=_ptr(winner))


def _case(D, H, G, B, seed):
    from test_gpu_parity import make_case

    L, idx, w, b, x, _ = make_case(D, H, G, 8, B, seed=seed, bias_std=0.2)
    return L, idx.to(DEV), w.to(DEV), b.to(DEV), x.to(DEV)


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")
@pytest.mark.parametrize("pool,k", [("sum", 0), ("topk_mean", 8)])
def test_static_forward_equals_gl_fwd_on_two_calls(pool, k):
    lib = N.library()
    spec = LevelSpec(pool, activation="relu", k=k) if pool == "topk_mean" else LevelSpec(pool, activation="relu")
    # the second call is smaller (fewer tokens, fewer pools); the first needs several passes of
    # the 64 MiB scratch for top-8 (partials of 2 x 8 x 4 bytes per chunk and token)
    for D, H, G, B, seed in ((2048, 1_000_000, 1000, 300, 1), (512, 40000, 40, 37, 2)):
        L, idx, w, b, x = _case(D, H, G, B, seed)
        rt = Level1Runtime(L, idx, spec, PhysicalPlan())
        outs = []
        for entry in ("gl_fwd", "gl_fwd_static"):
            pre = torch.full((B, G), float("nan"), device=DEV)
            win = torch.full((B, G, k), -7, device=DEV, dtype=torch.int32) if k else None
            a = _args(rt, x, w, b, pre, win, k, pool)
            ws = None
            if entry == "gl_fwd":
                need = lib.size_query("gl_fwd_workspace", a)
                ws = torch.empty(need, device=DEV, dtype=torch.uint8)
                a.ws, a.ws_bytes = _ptr(ws), need
            with torch.cuda.device(x.device):
                rc = getattr(lib.lib, entry)(ctypes.byref(a), ctypes.c_void_p(_stream(x.device)))
            assert rc == 0, f"{entry}: {lib.error(rc)}"
            torch.cuda.synchronize()
            outs.append((pre.cpu(), None if win is None else win.cpu()))
        (p1, w1), (p2, w2) = outs
        assert torch.equal(p1, p2), f"pre differs (D={D}, H={H}, B={B})"
        assert not torch.isnan(p2).any()
        if k:
            assert torch.equal(w1, w2), "topk_slot differs"


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")
def test_static_forward_orders_calls_on_two_streams():
    """Two calls on two streams of one GPU, issued back to back with no host synchronisation,
    share the static scratch; the library orders them (the second waits for the first's launches),
    so each gives gl_fwd's result."""
    lib = N.library()
    spec = LevelSpec("sum", activation="relu")
    cases = [_case(1024, 400_000, 400, 256, 3), _case(1024, 400_000, 400, 256, 4)]
    want, got = [], []
    for L, idx, w, b, x in cases:
        rt = Level1Runtime(L, idx, spec, PhysicalPlan())
        pre = torch.empty((x.shape[0], L.groups), device=DEV)
        a = _args(rt, x, w, b, pre)
        need = lib.size_query("gl_fwd_workspace", a)
        ws = torch.empty(need, device=DEV, dtype=torch.uint8)
        a.ws, a.ws_bytes = _ptr(ws), need
        assert lib.lib.gl_fwd(ctypes.byref(a), ctypes.c_void_p(_stream(x.device))) == 0
        want.append(pre)
        got.append((rt, x, w, b, torch.full_like(pre, float("nan"))))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s, (rt, x, w, b, pre) in zip(streams, got):
        a = _args(rt, x, w, b, pre)
        rc = lib.lib.gl_fwd_static(ctypes.byref(a), ctypes.c_void_p(s.cuda_stream))
        assert rc == 0, lib.error(rc)
    torch.cuda.synchronize()
    for (_, _, _, _, pre), ref in zip(got, want):
        assert torch.equal(pre, ref)


def test_static_forward_refuses_layers_beyond_the_scratch():
    """Host-side refusal (placeholder pointers never dereferenced): top-64 lists of 40,000 pools of
    256 slots take 2 KiB per chunk and 4-token tile, 78 MiB > 64 MiB."""
    lib = N.library()
    a = N.GlFwdArgs(X=16, idx=16, W=16, bias=16, counts=16, pre=16, B=8, D=64, G=40_000, S=256, K=8,
                    act=N.GL_ACT["identity"], pool=N.GL_POOL["topk_mean"], topk=64)
    assert lib.lib.gl_fwd_static(ctypes.byref(a), None) == N.GL_ERR_SCRATCH
    assert "static scratch" in lib.error(N.GL_ERR_SCRATCH)
