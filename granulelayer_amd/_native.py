"""ctypes binding of the HIP library (include/granulelayer_amd.h).

The library is loaded from ``granulelayer_amd/lib/libgranulelayer_amd.so`` (built in-tree by
``granulelayer_amd.build``).  At load the binding refuses a library whose ABI version or struct
layouts differ from the structures below, like the reference's native bridge
(sparse_pooling/backends/cuda/runtime.py:103-120, check_abi).  There is no fallback: every
entry point of the product path raises if the library is missing or refuses a call.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libgranulelayer_amd.so"
ABI_VERSION = 13

GL_ACT = {"identity": 0, "relu": 1, "gelu": 2}
GL_POOL = {"mean": 0, "sum": 1, "max": 2, "topk_mean": 3, "logmeanexp": 4, "power_mean": 5, "softmax_weighted": 6}
GL_DTYPE_F32, GL_DTYPE_BF16 = 0, 1
GL_ERR_SCRATCH = -8
FWD_STATIC_SCRATCH_BYTES = 64 << 20  # GL_FWD_STATIC_SCRATCH_BYTES

_P, _I32, _I64, _SZ, _F = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float


class GlFwdArgs(ctypes.Structure):
    _fields_ = [("X", _P), ("sxb", _I64), ("x_dtype", _I32), ("B", _I32), ("D", _I32), ("G", _I32), ("S", _I32),
                ("K", _I32), ("act", _I32), ("pool", _I32), ("topk", _I32), ("rec_shift", _I32), ("sps", _I32), ("gs", _I32), ("idx", _P), ("W", _P), ("bias", _P), ("counts", _P),
                ("sched", _P), ("win", _P), ("win_width", _I32), ("pre", _P), ("winner", _P), ("pool_param", _F),
                ("lse", _P), ("ws", _P), ("ws_bytes", _SZ), ("part_budget", _SZ), ("w_dtype", _I32),
                ("relu_mask", _P)]


class GlBwdArgs(ctypes.Structure):
    _fields_ = [("X", _P), ("sxb", _I64), ("x_dtype", _I32), ("B", _I32), ("D", _I32), ("G", _I32), ("S", _I32),
                ("K", _I32), ("act", _I32), ("pool", _I32), ("topk", _I32), ("rec_shift", _I32), ("sps", _I32), ("gs", _I32), ("idx", _P), ("W", _P), ("bias", _P), ("counts", _P),
                ("sched", _P), ("win", _P), ("win_width", _I32), ("g_pre", _P), ("winner", _P), ("pool_param", _F),
                ("pre", _P), ("lse", _P), ("dW", _P), ("db", _P),
                ("dX", _P), ("edges", _P), ("edges_bytes", _SZ),
                ("ws", _P), ("ws_bytes", _SZ), ("dz_budget", _SZ), ("w_dtype", _I32),
                ("relu_mask", _P)]


class GlEdgeArgs(ctypes.Structure):
    _fields_ = [("idx", _P), ("counts", _P), ("D", _I32), ("G", _I32), ("S", _I32), ("K", _I32), ("rec_shift", _I32),
                ("sps", _I32), ("gs", _I32), ("edges", _P),
                ("edges_bytes", _SZ), ("ws", _P), ("ws_bytes", _SZ)]


class GlAdamArgs(ctypes.Structure):
    _fields_ = [("p", _P), ("g", _P), ("m", _P), ("v", _P), ("n", _I64), ("moments_dtype", _I32), ("lr", _F),
                ("beta1", _F), ("beta2", _F), ("eps", _F), ("weight_decay", _F), ("bc1", _F), ("bc2", _F),
                ("p_dtype", _I32), ("stochastic", _I32), ("master", _P), ("seed", ctypes.c_uint64)]


class GlCoverArgs(ctypes.Structure):
    _fields_ = [("W", _P), ("a", _P), ("nvalid", _P), ("cand", _P), ("R", _I32), ("gpb", _I32), ("k", _I32),
                ("repair", _I32), ("importance", _P), ("env", _P), ("rec_idx", _P), ("W_out", _P), ("missing0", _P),
                ("swaps", _P), ("loss", _P), ("status", _P)]


STRUCTS = (GlFwdArgs, GlBwdArgs, GlEdgeArgs, GlAdamArgs, GlCoverArgs)  # gl_struct_layout ids 0..4
# every symbol include/granulelayer_amd.h declares
EXPORTS = ("gl_abi_version", "gl_struct_layout", "gl_error_string", "gl_fwd_workspace", "gl_fwd", "gl_fwd_static",
           "gl_fwd_mask_bytes",
           "gl_edges_size",
           "gl_edges_build", "gl_bwd_workspace", "gl_bwd", "gl_adam", "gl_sched_size", "gl_sched_build_host",
           "gl_sched_build", "gl_window_build_host", "gl_window_build", "gl_cover_select", "gl_trace_begin",
           "gl_trace_end")
KERNEL_NAMES = {1: "tile_x_kernel", 2: "fwd_kernel", 3: "fwd_finalize_kernel", 4: "c1t_kernel", 5: "bwd_w_kernel",
                6: "dx_kernel", 7: "dx_reduce_kernel", 8: "adam_kernel", 9: "edges_build", 10: "fwd_kernel_win",
                11: "bwd_w_kernel_win", 12: "max_events_dw_kernel", 13: "max_events_dx_kernel",
                14: "cover_select_kernel", 15: "sched_build_kernel", 16: "dx_dense_kernel",
                17: "dx_dma_kernel"}


class NativeError(RuntimeError):
    pass


def struct_layout(st) -> list:
    return [ctypes.sizeof(st)] + [getattr(st, name).offset for name, _ in st._fields_]


class Library:
    """One loaded copy of the HIP library with typed entry points."""

    def __init__(self, path: Path = LIB_PATH):
        if not Path(path).exists():
            raise NativeError(f"HIP library not found at {path}; build it with `python -m granulelayer_amd.build` "
                              "(the MI355X path has no CPU or PyTorch fallback)")
        self.path = Path(path)
        self.lib = ctypes.CDLL(str(path))
        L = self.lib
        L.gl_abi_version.restype = ctypes.c_int
        L.gl_struct_layout.restype = ctypes.c_int
        L.gl_struct_layout.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_longlong), ctypes.c_int]
        L.gl_error_string.restype = ctypes.c_char_p
        L.gl_error_string.argtypes = [ctypes.c_int]
        for name, st in (("gl_fwd", GlFwdArgs), ("gl_fwd_static", GlFwdArgs), ("gl_bwd", GlBwdArgs),
                         ("gl_edges_build", GlEdgeArgs), ("gl_adam", GlAdamArgs), ("gl_cover_select", GlCoverArgs)):
            f = getattr(L, name)
            f.restype, f.argtypes = ctypes.c_int, [ctypes.POINTER(st), _P]
        for name, st in (("gl_fwd_workspace", GlFwdArgs), ("gl_bwd_workspace", GlBwdArgs)):
            f = getattr(L, name)
            f.restype, f.argtypes = ctypes.c_int, [ctypes.POINTER(st), ctypes.POINTER(_SZ)]
        L.gl_trace_begin.restype = ctypes.c_int
        L.gl_trace_begin.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(_I32), ctypes.c_int]
        L.gl_trace_end.restype = ctypes.c_int
        L.gl_trace_end.argtypes = []
        L.gl_edges_size.restype = ctypes.c_int
        L.gl_edges_size.argtypes = [ctypes.POINTER(GlEdgeArgs), ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]
        L.gl_sched_size.restype = ctypes.c_int
        L.gl_sched_size.argtypes = [_I32, _I32, _I32, ctypes.POINTER(_SZ)]
        L.gl_sched_build_host.restype = ctypes.c_int
        L.gl_sched_build_host.argtypes = [_P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _P, _I32]
        L.gl_sched_build.restype = ctypes.c_int
        L.gl_sched_build.argtypes = [_P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P]
        L.gl_window_build.restype = ctypes.c_int
        L.gl_window_build.argtypes = [_P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P, _P]
        L.gl_window_build_host.restype = ctypes.c_int
        L.gl_window_build_host.argtypes = [_P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P, ctypes.POINTER(_I32)]
        self.check_abi()

    def check_abi(self):
        v = self.lib.gl_abi_version()
        if v != ABI_VERSION:
            raise NativeError(f"{self.path}: ABI version {v} != {ABI_VERSION} (stale library; rebuild)")
        for which, st in enumerate(STRUCTS):
            buf = (ctypes.c_longlong * 64)()
            n = self.lib.gl_struct_layout(which, buf, 64)
            want = struct_layout(st)
            if n != len(want) or list(buf[:n]) != want:
                raise NativeError(f"{self.path}: {st.__name__} layout mismatch (native {list(buf[:max(n, 0)])}, "
                                  f"binding {want})")

    def error(self, code: int) -> str:
        return self.lib.gl_error_string(code).decode()

    def call(self, name: str, *args):
        r = getattr(self.lib, name)(*args)
        if r != 0:
            raise NativeError(f"{name} failed (code {r}: {self.error(r)})")
        return r

    def size_query(self, name: str, args) -> int:
        out = _SZ(0)
        self.call(name, ctypes.byref(args), ctypes.byref(out))
        return int(out.value)

    def edges_size(self, args: GlEdgeArgs):
        e, w = _SZ(0), _SZ(0)
        self.call("gl_edges_size", ctypes.byref(args), ctypes.byref(e), ctypes.byref(w))
        return int(e.value), int(w.value)

    def sched_build(self, idx, counts, D: int, G: int, S: int, K: int, threads: int = 0, sps: int = 1, gs: int = 0):
        """Gather schedule (numpy uint32 array) from host int32 arrays idx [neurons, K] and counts [G]
        (G pools of S slots; sps > 1: the level-1 shards of G / sps groups of gs slots)."""
        import numpy as np

        idx = np.ascontiguousarray(idx, dtype=np.int32)
        counts = np.ascontiguousarray(counts, dtype=np.int32)
        rows = G * S if sps <= 1 else G // sps * gs
        if idx.size != rows * K or counts.size != G:
            raise ValueError("idx must hold one record per neuron and counts G entries")
        n = _SZ(0)
        self.call("gl_sched_size", G, S, K, ctypes.byref(n))
        out = np.empty(int(n.value) // 4, dtype=np.uint32)
        self.call("gl_sched_build_host", idx.ctypes.data, counts.ctypes.data, D, G, S, sps, gs, K, out.ctypes.data,
                  threads)
        return out

    def window_build(self, idx, counts, D: int, G: int, S: int, K: int, rec_shift: int = 0, sps: int = 1, gs: int = 0):
        """Per-pool input windows from host int32 arrays idx [neurons >> rec_shift, K] and counts [G]:
        (lo uint32 [G], widest window width)."""
        import numpy as np

        idx = np.ascontiguousarray(idx, dtype=np.int32)
        counts = np.ascontiguousarray(counts, dtype=np.int32)
        rows = G * S if sps <= 1 else G // sps * gs
        if idx.size != (rows >> rec_shift) * K or counts.size != G:
            raise ValueError("idx must hold one record per neuron (>> rec_shift) and counts G entries")
        lo = np.empty(G, dtype=np.uint32)
        width = _I32(0)
        self.call("gl_window_build_host", idx.ctypes.data, counts.ctypes.data, D, G, S, sps, gs, K, rec_shift,
                  lo.ctypes.data, ctypes.byref(width))
        return lo, int(width.value)


class KernelTrace:
    """Per-kernel GPU time of the library's launches inside a ``with`` block, from HIP events
    recorded around every launch on its own stream (gl_trace_begin / gl_trace_end).

        with KernelTrace(max_launches=64) as tr:
            ...                                # library calls
        tr.times_ms()  -> {"fwd_kernel": [ms, ...], ...}
    """

    def __init__(self, max_launches: int = 256, lib: "Library" = None):
        import torch

        self.lib = lib or library()
        self.events = [torch.cuda.Event(enable_timing=True) for _ in range(2 * max_launches)]
        for e in self.events:  # torch creates the HIP event on its first record
            e.record()
        torch.cuda.synchronize()
        self._handles = (ctypes.c_void_p * (2 * max_launches))(*[e.cuda_event for e in self.events])
        self._ids = (_I32 * max_launches)()
        self.n = 0
        self.max = max_launches

    def __enter__(self):
        for e in self.events:  # materialise the HIP events
            if e.cuda_event == 0:
                raise NativeError("torch event not created")
        self.lib.call("gl_trace_begin", self._handles, self._ids, self.max)
        return self

    def __exit__(self, *exc):
        self.n = self.lib.lib.gl_trace_end()
        return False

    def times_ms(self) -> dict:
        import torch

        torch.cuda.synchronize()
        out = {}
        for i in range(self.n):
            name = KERNEL_NAMES.get(int(self._ids[i]), str(int(self._ids[i])))
            out.setdefault(name, []).append(self.events[2 * i].elapsed_time(self.events[2 * i + 1]))
        return out


_lock = threading.Lock()
_library = None


def library() -> Library:
    """The process-wide library (loaded on first use)."""
    global _library
    with _lock:
        if _library is None:
            _library = Library()
        return _library
