"""The C-ABI library loads and exports every symbol include/granulelayer_amd.h declares; the
ctypes structures match the native layouts; argument refusal happens before any device use.
Runs on the CPU (no compute calls)."""
import ctypes
import re
from pathlib import Path

import pytest

from granulelayer_amd import _native as N

HEADER = Path(__file__).resolve().parents[1] / "include" / "granulelayer_amd.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(gl_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_binding_exports():
    assert declared_functions() == sorted(N.EXPORTS)


def test_library_loads_and_exports_every_declared_symbol():
    lib = N.library()
    for name in declared_functions():
        assert hasattr(lib.lib, name), name
    assert lib.lib.gl_abi_version() == N.ABI_VERSION


@pytest.mark.parametrize("which", range(len(N.STRUCTS)))
def test_struct_layouts_match(which):
    lib = N.library()
    buf = (ctypes.c_longlong * 64)()
    n = lib.lib.gl_struct_layout(which, buf, 64)
    assert list(buf[:n]) == N.struct_layout(N.STRUCTS[which])


def test_abi_check_rejects_a_shifted_struct(monkeypatch):
    """A binding whose struct differs from the library's must refuse to load (the reference's
    test_device_runtime.py:136-151 pattern)."""

    class Shifted(ctypes.Structure):
        _fields_ = [("pad", ctypes.c_int32)] + list(N.GlFwdArgs._fields_)

    monkeypatch.setattr(N, "STRUCTS", (Shifted,) + N.STRUCTS[1:])
    with pytest.raises(N.NativeError, match="layout mismatch"):
        N.Library()


def test_unknown_struct_and_error_strings():
    lib = N.library()
    assert lib.lib.gl_struct_layout(99, None, 0) < 0
    for code in (0, -1, -2, -3, -4, -5, -7):
        assert lib.error(code)


def test_arguments_are_refused_before_device_use():
    lib = N.library()
    a = N.GlFwdArgs(B=4, D=64, G=2, S=32, K=8)  # null pointers
    out = ctypes.c_size_t()
    assert lib.lib.gl_fwd_workspace(ctypes.byref(a), ctypes.byref(out)) == -1
    assert lib.lib.gl_fwd(ctypes.byref(a), None) == -1
    b = N.GlBwdArgs(B=4, D=64, G=2, S=32, K=8)
    assert lib.lib.gl_bwd(ctypes.byref(b), None) == -1
    e = N.GlEdgeArgs(D=64, G=2, S=32, K=12)
    assert lib.lib.gl_edges_size(ctypes.byref(e), ctypes.byref(out), ctypes.byref(out)) == -2
    m = N.GlAdamArgs(n=-1)
    assert lib.lib.gl_adam(ctypes.byref(m), None) == -1
    m = N.GlAdamArgs(n=0)
    assert lib.lib.gl_adam(ctypes.byref(m), None) == 0


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(N.NativeError, match="not found"):
        N.Library(tmp_path / "nope.so")


def test_pool_limits_are_refused_by_the_size_query():
    """Top-k mean takes k a power of two in [1, 64] (the reference's LevelSpec check) and pools of
    up to 4096 slots; other pool codes are refused.  Host-side checks only: the pointers are
    placeholders that the size query never dereferences."""
    lib = N.library()
    out = ctypes.c_size_t()

    def query(pool, topk, S):
        a = N.GlFwdArgs(X=16, idx=16, W=16, bias=16, counts=16, B=8, D=64, G=2, S=S, K=8,
                        act=N.GL_ACT["identity"], pool=pool, topk=topk)
        return lib.lib.gl_fwd_workspace(ctypes.byref(a), ctypes.byref(out))

    tk = N.GL_POOL["topk_mean"]
    for k in (1, 2, 8, 64):
        assert query(tk, k, 4096) == 0 and out.value > 0
    for k in (0, 3, 12, 128):
        assert query(tk, k, 256) == -1
    assert query(tk, 8, 4097) == -2
    assert query(N.GL_POOL["max"], 0, 100000) == 0
    assert query(7, 0, 256) == -2


def test_forward_workspace_is_bounded_as_the_batch_grows():
    """The forward runs token chunks whose partial results fit part_budget (default 8 GiB), so its
    workspace stops growing with B: at the C2 shape with top-16 mean, B = 8192 needs no more than
    B = 1024; sum pooling at B = 256 (the headline) still runs as one pass.  Host-side size query
    only (placeholder pointers, never dereferenced)."""
    lib = N.library()
    out = ctypes.c_size_t()

    def ws(B, pool, topk=0, budget=0, D=4096):
        a = N.GlFwdArgs(X=16, idx=16, W=16, bias=16, counts=16, B=B, D=D, G=98_304, S=1024, K=8,
                        act=N.GL_ACT["relu"], pool=N.GL_POOL[pool], topk=topk, part_budget=budget)
        assert lib.lib.gl_fwd_workspace(ctypes.byref(a), ctypes.byref(out)) == 0
        return out.value

    tk = [ws(B, "topk_mean", 16) for B in (1024, 8192, 65536)]
    assert tk[0] == tk[1] == tk[2] <= (8 << 30) + 1024 * 4096 * 4 + 512
    assert ws(256, "sum") == 256 * 4096 * 4 + 98_304 * 4 * 256 * 4  # X tiles + one pass of partials
    assert ws(1 << 20, "max") <= (8 << 30) + (1 << 20) * 4096 * 4
    small = ws(1 << 16, "sum", budget=64 << 20)
    assert small <= (64 << 20) + (1 << 16) * 4096 * 4
    # a budget below one token tile's partials still runs (one tile per pass)
    assert ws(64, "topk_mean", 64, budget=1) == 4 * 4096 * 4 + 2 * 98_304 * 4 * 4 * 64 * 4


def test_pool_geometry_is_validated_by_the_size_queries():
    """sps / gs (two-level pooling's level-1 shards): sps <= 1 means the pools are the groups and a
    given gs must equal S; sps > 1 needs G a multiple of sps and (sps - 1) S < gs <= sps S, so every
    shard starts inside its group.  Host-side checks of gl_fwd_workspace, gl_bwd_workspace and
    gl_edges_size (placeholder pointers, never dereferenced)."""
    lib = N.library()
    out, e, w = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()

    def q(sps, gs, G=16, S=256, rec_shift=0):
        kw = dict(X=16, idx=16, W=16, bias=16, counts=16, B=8, D=64, G=G, S=S, K=8, act=N.GL_ACT["relu"],
                  pool=N.GL_POOL["mean"], sps=sps, gs=gs, rec_shift=rec_shift)
        f = lib.lib.gl_fwd_workspace(ctypes.byref(N.GlFwdArgs(**kw)), ctypes.byref(out))
        b = lib.lib.gl_bwd_workspace(ctypes.byref(N.GlBwdArgs(**kw)), ctypes.byref(out))
        ea = N.GlEdgeArgs(idx=16, counts=16, D=64, G=G, S=S, K=8, sps=sps, gs=gs, rec_shift=rec_shift)
        x = lib.lib.gl_edges_size(ctypes.byref(ea), ctypes.byref(e), ctypes.byref(w))
        assert f == b == x, (f, b, x)
        return f

    assert q(0, 0) == 0 and q(1, 0) == 0 and q(1, 256) == 0
    assert q(1, 384) == -1 and q(0, 512) == -1  # groups are not pools of S slots
    assert q(2, 384) == 0 and q(2, 512) == 0 and q(4, 1000) == 0
    assert q(2, 256) == -1 and q(2, 513) == -1  # the second shard would start outside / end past the group
    assert q(3, 600, G=16) == -1  # G not a multiple of sps
    assert q(-1, 0) == -1
    assert q(2, 384, S=256, rec_shift=4) == -2  # shared index records are not sharded


def test_an_explicit_workspace_budget_is_honoured():
    """workspace_budget=None leaves the library its defaults (8 GiB of forward partials, 64 GiB of
    smooth-pool dz); any explicit value, the reference's own 512 MiB default included, is what the
    launches are given, and it bounds gl_bwd_workspace of a smooth pool at the C2 shape.  Host-side
    only (CPU runtime objects, placeholder pointers never dereferenced)."""
    import torch

    from granulelayer_amd import backend as BK
    from granulelayer_amd.autograd import Level1Runtime
    from granulelayer_amd.config import DEFAULT_WORKSPACE_BUDGET, LevelSpec, PhysicalPlan
    from granulelayer_amd.layout import SparseLayout

    L = SparseLayout(256, 4096, 4, 8, 8, False)
    idx = torch.zeros(L.index_shape, dtype=torch.int32)
    lv = LevelSpec(type="logmeanexp")
    default = Level1Runtime(L, idx, lv, PhysicalPlan())
    explicit = Level1Runtime(L, idx, lv, PhysicalPlan(), workspace_budget=DEFAULT_WORKSPACE_BUDGET)
    assert BK.HipBackend.part_budget(default) == 0 and BK.HipBackend.dz_budget(default) == BK.DZ_BUDGET
    assert BK.HipBackend.part_budget(explicit) == DEFAULT_WORKSPACE_BUDGET
    assert BK.HipBackend.dz_budget(explicit) == DEFAULT_WORKSPACE_BUDGET
    for bad in (0, -1, 1.5, True):
        with pytest.raises(ValueError):
            Level1Runtime(L, idx, lv, PhysicalPlan(), workspace_budget=bad)

    lib = N.library()
    out = ctypes.c_size_t()

    def bwd_ws(dz_budget, B=1024):
        # 1,048,576 neurons: 4 MiB of dz per token
        a = N.GlBwdArgs(X=16, idx=16, W=16, bias=16, counts=16, g_pre=16, pre=16, lse=16, dW=16, db=16, dX=16,
                        edges=16, B=B, D=1024, G=4096, S=256, K=8, act=N.GL_ACT["identity"],
                        pool=N.GL_POOL["logmeanexp"], pool_param=1.0, dz_budget=dz_budget)
        assert lib.lib.gl_bwd_workspace(ctypes.byref(a), ctypes.byref(out)) == 0
        return out.value

    big, small = bwd_ws(BK.DZ_BUDGET), bwd_ws(DEFAULT_WORKSPACE_BUDGET)
    # 1024-token chunks (4 GiB of dz) without a budget, 128-token chunks (512 MiB) with 512 MiB;
    # the rest of the workspace (X tiles, coefficients, dX partials) scales with the chunk too
    assert big - small >= (1024 - 128) * (4 << 20)
    assert small - bwd_ws(DEFAULT_WORKSPACE_BUDGET, B=128) < (1 << 20)  # B = 128: the same one chunk
    assert bwd_ws(DEFAULT_WORKSPACE_BUDGET // 2) < small


def test_relu_bit_sizes_follow_the_layer():
    """gl_fwd_mask_bytes: G x ceil(S / 256) chunks x ceil(B / 4) tiles x 64 lanes x 2 bytes for ReLU
    mean / sum at fan-in 8 with 4-token tiles; 0 for the layers without bits (fp32 X over
    4097..8192 inputs runs two-token tiles, fan-in 16, other activations or pools, shared records)."""
    lib = N.library()

    def size(**kw):
        a = N.GlFwdArgs(**{"B": 300, "D": 1024, "G": 64, "S": 1024, "K": 8, "act": N.GL_ACT["relu"],
                           "pool": N.GL_POOL["sum"], **kw})
        return lib.size_query("gl_fwd_mask_bytes", a)

    assert size() == 64 * 4 * 75 * 128
    assert size(B=301, S=1000) == 64 * 4 * 76 * 128
    assert size(pool=N.GL_POOL["mean"], D=6000, x_dtype=N.GL_DTYPE_BF16) == 64 * 4 * 75 * 128
    assert size(D=12000) == 64 * 4 * 75 * 128
    assert size(D=6000) == 0
    assert size(K=16) == 0
    assert size(act=N.GL_ACT["gelu"]) == 0
    assert size(pool=N.GL_POOL["max"]) == 0
    assert size(rec_shift=4) == 0


def test_lds_probe_library_is_separate_and_refuses_bad_shapes():
    """bench.py --lds-probe's kernel lives in its own library: the layer's library does not export
    it, and the probe refuses an unsupported slot size or launch shape before any device use."""
    from granulelayer_amd.build import PROBE_LIB

    if not PROBE_LIB.exists():
        pytest.skip("probe library not built")
    probe = ctypes.CDLL(str(PROBE_LIB))
    probe.gl_lds_probe.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                   ctypes.c_void_p]
    buf = ctypes.create_string_buffer(64)
    assert probe.gl_lds_probe(4, buf, 1, buf, 1, None) == -1
    assert probe.gl_lds_probe(16, buf, 0, buf, 1, None) == -1
    assert probe.gl_lds_probe(16, None, 1, buf, 1, None) == -1
    assert not hasattr(N.library().lib, "gl_lds_probe")
