"""Benchmark of the MI355X sparse projection-and-pool layer (one JSON line on stdout).

Workload (BASELINE.json metric "train-step ms & G edge-MAC/s at 100M neurons fan-in 8, B=256"):
one training step of the C2-shaped layer -- N = 100,663,296 neurons, fan-in 8, D = 4096 inputs,
B = 256 tokens, pools of 1024 (G = 98,304), ReLU + sum pooling, fp32 X / W / moments -- made of
the fused forward, the recompute backward (dX, dW and db into fp32 main_grad) and the fused
AdamW step (lr 1e-3, betas 0.9/0.999, eps 1e-8, wd 0).  Synthetic seeded data: indices uniform
and distinct per neuron, W ~ N(0, 1/8), bias 0, X and dY ~ N(0, 1).  The forward-only time of the
same layer (the headline forward) is reported beside it.

value = useful edge-MACs per second of the whole step (B * N * 8 / step time, one pass, as the
reference's useful_tflops(passes=1), sparse_pooling/benchmarks/common.py:80-82).

Usage: python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--no-cpu-baseline] [--no-extra]
                      [--relu-bits keep|recompute]

The layers run with PhysicalPlan(relu_bits="keep") by default: the forward keeps one ReLU bit per
(token, neuron) (1/32 of the hidden tensor's fp32 bytes) and the backward's dW pass reads it
instead of recomputing z, with the same results bit for bit.  The same step with the reference's
recompute (relu_bits="recompute") is timed beside it ("other_relu_bits").

Beside the headline the line carries: the C1 train step on the GPU, the C4
full training step (configs[3], 3 timed steps), the one-time layer setup, and cpu_baseline = the
reference's CPU path on C1 timed on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# MI355X published peaks
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3

CFG = dict(N=100_663_296, K=8, D=4096, B=256, pool=1024)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def algorithmic(kernel: str, B: int, N: int, K: int, D: int, G: int, x_bytes: int = 4, relu_bits: bool = False):
    """(bytes, flops) of one training step's launches of a kernel (one launch each, except the
    AdamW kernel: one launch for the weights, one for the bias): every input read once, every
    output written once.  relu_bits: the forward also writes the ReLU bits (N B / 8 bytes) and the
    dW pass reads them instead of W, bias and the z recompute (its flops are dW's 2 B E alone)."""
    E = N * K
    if kernel == "fwd_kernel":
        # idx + W + bias, X once, pooled output (+ the ReLU bits)
        return 4 * E + 4 * E + 4 * N + B * D * x_bytes + 4 * B * G + (N * B // 8 if relu_bits else 0), 2 * B * E
    if kernel == "bwd_w_kernel":
        if relu_bits:  # idx, X once, the forward's bits, dW/db read-modify-write, mask bits written
            return 4 * E + B * D * x_bytes + N * B // 8 + 8 * E + 8 * N + N * B // 8, 2 * B * E
        # idx + W + bias, X once, dW/db read-modify-write, mask bits written
        return 4 * E + 4 * E + 4 * N + B * D * x_bytes + 8 * E + 8 * N + N * B // 8, 4 * B * E
    if kernel in ("dx_kernel", "dx_dma_kernel"):
        # per edge: record, weight and the neuron's B mask bits; dX written once
        return E * (4 + 4 + B // 8) + 4 * B * D, 2 * B * E
    if kernel == "adam_kernel":
        return 32 * (E + N), 12 * (E + N)
    if kernel == "bwd_smooth_kernel":
        # as bwd_w_kernel, with every neuron's dz row (fp32 per token) written instead of mask bits
        return 4 * E + 4 * E + 4 * N + B * D * x_bytes + 8 * E + 8 * N + 4 * N * B, 4 * B * E
    if kernel == "dx_dense_kernel":
        # per edge: record, weight and the neuron's dz row; dX written once
        return E * (4 + 4 + 4 * B) + 4 * B * D, 2 * B * E
    return None, None


# --pooling choices: (pooling spec of the layer, description in the bench line)
POOLINGS = {
    "sum": ("sum", "sum(relu)"),
    "mean": ("mean", "mean(relu)"),
    "max": ("max", "relu(max z)"),
    "topk": ({"type": "topk_mean", "k": 8}, "top-8 mean(z)"),
    "lme": ({"type": "logmeanexp", "temperature": 1.0, "activation": "relu"}, "logmeanexp(relu, tau 1)"),
    "power": ({"type": "power_mean", "p": 2.0, "activation": "relu"}, "power mean(relu, p 2)"),
    "softmax": ({"type": "softmax_weighted", "beta": 1.0, "activation": "relu"}, "softmax-weighted(relu, beta 1)"),
    "two_level": ({"levels": [{"type": "mean", "neurons_per_shard": 256}, {"type": "logmeanexp"}]},
                  "mean(relu) over shards of 256, then logmeanexp over 4 shards"),
}

CONFIG_WORK = {"C1": "fwd+bwd+adam", "C2": "fwd", "C3": "fwd+bwd", "C4": "fwd+bwd+adam", "C5": "fwd+bwd"}


def run_config(name: str, steps: int, warmup: int):
    """One JSON line for a BASELINE config at its full size: the config's own work (forward,
    forward + backward, or the training step) timed over ``steps`` calls after ``warmup``."""
    import torch

    from granulelayer_amd import FusedAdamW, SparsePoolingLayer
    from granulelayer_amd._native import KernelTrace
    from granulelayer_amd.synthetic import CONFIGS, make_problem

    c = CONFIGS[name]
    work = CONFIG_WORK[name]
    dev = torch.device("cuda", 0)
    N, K, D, B, pool = c["N"], c["K"], c["D"], c["B"], c["pool"]
    G = N // pool
    t0 = time.time()
    lay = SparsePoolingLayer(D, N, G, fan_in=K, shared_neurons=None, pooling="sum", dtype=torch.float32, device=dev,
                             plan=_plan(),
                             seed=0)
    if c["indices"] != "uniform":  # locality windows (C3) or top-16 of 64 candidates (C5)
        pr = make_problem(name, device=dev, seed=0)
        with torch.no_grad():
            lay.indices.copy_(pr.idx)
            lay.weight.copy_(pr.w)
        del pr
    lay.enable_main_grad()
    opt = FusedAdamW(lay.parameters(), lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, moments="fp32")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    x = torch.randn(B, D, generator=gen, device=dev).to(c["x_dtype"])
    dy = torch.randn(B, G, generator=gen, device=dev).to(c["x_dtype"]).float()
    torch.cuda.synchronize()
    log(f"{name}: layer N={N:,} K={K} D={D} B={B} pool={pool} ready in {time.time() - t0:.1f} s")

    def one():
        if work == "fwd":
            with torch.no_grad():
                lay(x)
            return
        y = lay(x)
        y.backward(dy)
        if work.endswith("adam"):
            opt.step()
        else:
            lay.zero_main_grad()

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with KernelTrace(max_launches=128 * steps) as tr:
        e0.record()
        for _ in range(steps):
            one()
        e1.record()
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    kt = {k: round(sum(v) / len(v), 4) for k, v in tr.times_ms().items()}
    out = {"metric": f"BASELINE config {name} ({work}) ms and G edge-MAC/s", "config": name, "work": work,
           "value": round(B * N * K / (ms * 1e-3) / 1e9, 2), "unit": "G edge-MAC/s", "ms": round(ms, 3),
           "steps": steps, "warmup": warmup, "neurons": N, "fan_in": K, "d_in": D, "batch": B, "pool": pool,
           "x_dtype": str(c["x_dtype"]).replace("torch.", ""), "indices": c["indices"], "kernels_ms": kt}
    print(json.dumps(out), flush=True)


def _med_iqr(v):
    import numpy as np

    q1, q2, q3 = np.percentile(np.asarray(v, dtype=np.float64), [25, 50, 75])
    return round(q2 * 1e3, 2), round((q3 - q1) * 1e3, 2)


# PhysicalPlan.relu_bits of every layer the bench builds ("keep": the forward keeps its ReLU bits
# for the backward's dW pass; "recompute": the reference's O(B x G) checkpoint); --relu-bits
RELU_BITS = "keep"


def _plan():
    from granulelayer_amd import PhysicalPlan

    return PhysicalPlan(relu_bits=RELU_BITS)


def lds_patterns(bytes_: int, kind: str, rng) -> "np.ndarray":
    """Byte offsets into a 64-KiB LDS tile for 8 reads x 64 lanes of one gather pattern.

    A bank row is 256 bytes (64 banks of 4 bytes), so a 16-byte slot's residue is slot mod 16 and an
    8-byte slot's is slot mod 32; `kind` fixes the residue each lane reads, the row is random."""
    import numpy as np

    nres = 256 // bytes_
    nrow = 65536 // 256
    out = np.empty((8, 64), dtype=np.uint32)
    for r in range(8):
        if kind == "linear":  # lane l reads slot l: every bank once per 256 bytes
            res = np.arange(64) % nres
            rows = np.arange(64) // nres
        else:
            rows = rng.integers(0, nrow, 64)
            if kind == "random":
                res = rng.integers(0, nres, 64)
            elif kind == "rows_distinct":  # each 16-lane row a permutation of 16 residues
                res = np.concatenate([rng.permutation(nres)[:16] for _ in range(4)])
            elif kind in ("rows_matched", "rows_matched_swapped"):
                # lanes 16-31 read the residue set of lanes 0-15 per 4-lane block (any order), and
                # lanes 48-63 that of lanes 32-47; rows distinct
                res = np.empty(64, dtype=np.int64)
                for h in (0, 32):
                    a = rng.permutation(nres)[:16]
                    b = np.concatenate([rng.permutation(a[4 * k:4 * k + 4]) for k in range(4)])
                    if kind == "rows_matched_swapped":  # blocks 0 and 1 of the second row trade sets
                        b = np.concatenate([b[4:8], b[0:4], b[8:]])
                    res[h:h + 16], res[h + 16:h + 32] = a, b
            elif kind == "halves_distinct":  # each 32-lane half a permutation of 32 residues
                res = np.concatenate([rng.permutation(nres)[:32] for _ in range(2)])
            elif kind == "halves_one_repeat":  # the same with one residue read twice in each half
                hs = []
                for _ in range(2):
                    h = rng.permutation(nres)[:32]
                    h[31] = h[0]
                    hs.append(h)
                res = np.concatenate(hs)
            elif kind == "rows16_colliding":  # 16-lane rows distinct, both rows of a half the same 16
                hs = []
                for _ in range(2):
                    a = rng.permutation(nres)[:16]
                    hs += [a, rng.permutation(a)]
                res = np.concatenate(hs)
            else:
                raise ValueError(kind)
        out[r] = (rows * 256 + res * bytes_).astype(np.uint32)
    return out


def lds_probe(iters: int = 20000):
    """`bench.py --lds-probe`: one workgroup of 16 waves per CU reads 8 independent patterns per
    loop iteration with ds_read_b128 (16-byte slots) or ds_read_b64 (8-byte slots); prints bytes
    per shader clock per CU (median over the workgroups) for each lane-to-bank pattern."""
    import ctypes

    import numpy as np
    import torch

    from granulelayer_amd.build import PROBE_LIB

    if not PROBE_LIB.exists():
        raise SystemExit(f"{PROBE_LIB} is missing: run __graft_entry__.build() first")
    lib = ctypes.CDLL(str(PROBE_LIB))
    lib.gl_lds_probe.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                 ctypes.c_void_p]
    dev = torch.device("cuda", 0)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    rng = np.random.default_rng(0)
    stream = torch.cuda.current_stream(dev).cuda_stream
    cases = [(16, k) for k in ("linear", "random", "rows_distinct", "rows_matched", "rows_matched_swapped")]
    cases += [(8, k) for k in ("linear", "random", "halves_distinct", "halves_one_repeat", "rows16_colliding")]
    rows = []
    for bytes_, kind in cases:
        offs = torch.from_numpy(lds_patterns(bytes_, kind, rng).astype(np.int32)).to(dev)
        cyc = torch.zeros(cus * 16, dtype=torch.int64, device=dev)
        for _ in range(2):  # the first launch warms up
            rc = lib.gl_lds_probe(bytes_, offs.data_ptr(), iters, cyc.data_ptr(), cus, stream)
            if rc != 0:
                raise SystemExit(f"gl_lds_probe failed ({bytes_}, {kind})")
        torch.cuda.synchronize()
        per_wg = cyc.view(cus, 16).max(dim=1).values.double().cpu().numpy()
        rate = 16 * iters * 8 * 64 * bytes_ / per_wg
        rows.append({"slot_bytes": bytes_, "pattern": kind, "B_per_clk_per_CU": round(float(np.median(rate)), 1),
                     "min": round(float(rate.min()), 1), "max": round(float(rate.max()), 1)})
        print(json.dumps(rows[-1]), flush=True)
    print(json.dumps({"lds_probe": rows, "cus": cus, "iters": iters, "waves_per_cu": 16, "reads_per_iter": 8}),
          flush=True)


def c1_problem():
    """BASELINE configs[0] (the reference's CPU-runnable case): B=64, D=1024, N=1,048,576, fan-in 8,
    pools of 256, seed 0, generated on the CPU so the GPU and the CPU path see the same bits."""
    from granulelayer_amd.synthetic import make_problem

    return make_problem("C1", device="cpu", seed=0)


def c1_gpu(pr, steps: int, warmup: int):
    """The C1 training step (forward, recompute backward into main_grad, FusedAdamW) on the GPU,
    with the layer's first output and input gradient for the CPU comparison."""
    import torch

    from granulelayer_amd import FusedAdamW, SparsePoolingLayer

    L = pr.layout
    dev = torch.device("cuda", 0)
    lay = SparsePoolingLayer(L.input_dim, L.hidden_dim, L.groups, fan_in=L.fan_in, shared_neurons=None, plan=_plan(),
                             pooling="sum", dtype=torch.float32, device=dev, seed=0)
    with torch.no_grad():
        lay.indices.copy_(pr.idx.to(dev))
        lay.weight.copy_(pr.w.to(dev))
        lay.bias.copy_(pr.b.to(dev))
    lay.enable_main_grad()
    opt = FusedAdamW(lay.parameters(), lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, moments="fp32")
    x = pr.x.to(dev).requires_grad_(True)
    dy = pr.dy.to(dev)
    y = lay(x)
    y.backward(dy)
    first = (y.detach().cpu(), x.grad.detach().cpu())
    opt.step()

    def step():
        y = lay(x)
        y.backward(dy)
        opt.step()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    del lay, opt
    return ms, first


def cpu_baseline(pr, steps: int, gpu_first):
    """The reference's CPU path on BASELINE configs[0] (C1): the materialising torch restatement of
    sparse_pooling/reference (oracle/reference_port.py) with torch.optim.Adam, timed on the host
    cores; its first output and input gradient are compared with the GPU's on the same inputs."""
    import torch

    from oracle.reference_port import PortStep

    st = PortStep(pr.idx, pr.w, pr.b, pr.layout.counts_tensor("cpu"), pr.layout.slots_per_group, pool="sum")
    x = pr.x.float().detach().requires_grad_(True)
    y = st.forward(x)
    (y * pr.dy).sum().backward()
    gy, gdx = gpu_first
    rel = lambda a, b: float((a.double() - b.double()).norm() / b.double().norm())  # noqa: E731
    parity = {"y_rel_err": rel(gy, y.detach()), "dx_rel_err": rel(gdx, x.grad)}
    st.w.grad = None
    st.b.grad = None
    times = [st.step(pr.x.float(), pr.dy) for _ in range(steps)]
    macs = pr.B * pr.edges
    step_med, step_iqr = _med_iqr([t["step"] for t in times])
    out = {"value": round(macs / (step_med * 1e-3) / 1e9, 4), "unit": "G edge-MAC/s",
           "cores": torch.get_num_threads(), "kind": "port",
           "sample": (f"BASELINE configs[0] (C1) whole: train step (fwd + bwd + torch.optim.Adam) of B=64, D=1024, "
                      f"N=1,048,576, fan-in 8, pools of 256, seed 0, in the materialising torch restatement of "
                      f"sparse_pooling/reference on the host; {steps} timed steps after one untimed step; "
                      f"cpu: {cpu_model()}, os.cpu_count()={os.cpu_count()}"),
           "ms_step_median": step_med, "ms_step_iqr": step_iqr, "parity_vs_gpu": parity}
    for k in ("fwd", "bwd", "adam"):
        out[f"ms_{k}_median"], out[f"ms_{k}_iqr"] = _med_iqr([t[k] for t in times])
    return out


def c4_step(steps: int, warmup: int):
    """BASELINE configs[3] (C4): the full training step at N=100,663,296, D=8192, B=1024, bf16 X,
    uniform indices, fwd + recompute bwd + FusedAdamW (fp32 moments), with per-kernel times."""
    import torch

    from granulelayer_amd import FusedAdamW, SparsePoolingLayer
    from granulelayer_amd._native import KernelTrace
    from granulelayer_amd.synthetic import CONFIGS

    c = CONFIGS["C4"]
    N, K, D, B, pool = c["N"], c["K"], c["D"], c["B"], c["pool"]
    G = N // pool
    dev = torch.device("cuda", 0)
    lay = SparsePoolingLayer(D, N, G, fan_in=K, shared_neurons=None, pooling="sum", dtype=torch.float32, device=dev,
                             plan=_plan(),
                             seed=0)
    lay.enable_main_grad()
    opt = FusedAdamW(lay.parameters(), lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, moments="fp32")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    x = torch.randn(B, D, generator=gen, device=dev).to(torch.bfloat16)
    dy = torch.randn(B, G, generator=gen, device=dev).to(torch.bfloat16).float()
    setup = setup_times(lay, x)

    def step():
        y = lay(x)
        y.backward(dy)
        opt.step()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with KernelTrace(max_launches=128 * steps) as tr:
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    kt = {k: round(sum(v) / steps, 3) for k, v in tr.times_ms().items()}
    del lay, opt
    torch.cuda.empty_cache()
    return {"workload": "BASELINE configs[3] (C4): fwd + recompute bwd (dX, dW, db) + FusedAdamW, N=100,663,296, "
                        "fan-in 8, D=8192, B=1024, pools of 1024, bf16 X, fp32 W and moments",
            "ms_per_step": round(ms, 3), "steps": steps, "warmup": warmup,
            "G_edge_macs_per_s": round(B * N * K / (ms * 1e-3) / 1e9, 2), "kernels_ms_per_step": kt, "setup": setup}


def setup_times(lay, x):
    """One-time layer setup the first training step pays, timed explicitly: the gather schedule
    (host build from a device-to-host copy of the indices, then upload), the pool windows (host),
    and the input-major edge list (GPU)."""
    import torch

    from granulelayer_amd.backend import HipBackend

    be = HipBackend.get()
    rt = lay._runtime()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    be.schedule(rt)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    be.windows(rt)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    be.edges(rt)
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    return {"gather_schedule_ms": round((t1 - t0) * 1e3, 1), "pool_windows_ms": round((t2 - t1) * 1e3, 1),
            "edge_list_ms": round((t3 - t2) * 1e3, 1), "total_ms": round((t3 - t0) * 1e3, 1)}


def read_profile(path: str) -> dict:
    """Per kernel, from a committed rocprofv3 summary: ``traffic <kernel> <bytes>`` (calibrated HBM
    bytes per dispatch: FETCH_SIZE and WRITE_SIZE, each scaled by what the counter reads for a device
    copy of known size) and ``profile_ms <kernel> <ms>`` (the kernel's average duration in the same
    profiled command)."""
    out = {}
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] in ("traffic", "profile_ms"):
                    out.setdefault(parts[1], {})[parts[0]] = float(parts[2])
    except OSError:
        pass
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--relu-bits", choices=("keep", "recompute"), default="keep",
                    help="PhysicalPlan.relu_bits of the timed layers (the other mode's step is timed beside it)")
    ap.add_argument("--cpu-steps", type=int, default=5, help="timed steps of the C1 CPU baseline (after one untimed)")
    ap.add_argument("--no-extra", action="store_true", help="skip the C1 and C4 extra measurements")
    ap.add_argument("--config", choices=sorted(CONFIG_WORK), default=None,
                    help="time one BASELINE config's own work at full size instead of the headline step")
    ap.add_argument("--pooling", choices=sorted(POOLINGS), default="sum",
                    help="pooling of the train-step layer (default: the headline's sum of relu; max: the "
                         "reference's defaults, relu(max z), winners saved for backward; topk: top-8 mean, "
                         "slots saved; lme / power / softmax: the smooth operators; two_level: mean over "
                         "shards of 256, then LogMeanExp over the 4 shard features)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (calibrates rocprofv3 byte counters)")
    ap.add_argument("--lds-probe", action="store_true",
                    help="only measure the LDS gather rate (ds_read_b128 / ds_read_b64) of lane-to-bank patterns")
    args = ap.parse_args()
    global RELU_BITS
    RELU_BITS = args.relu_bits
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build measures one MI355X (--gpus {args.gpus} requested); "
              "nothing in it shards across GPUs", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    if args.config:
        run_config(args.config, args.steps, args.warmup)
        return
    if args.lds_probe:
        lds_probe()
        return
    if args.copy_probe:
        n = args.copy_probe * (1 << 20) // 4
        a = torch.ones(n, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)  # runtime copy kernel
        for _ in range(3):
            torch.mul(a, 1.0, out=b)  # elementwise kernel reading and writing the same bytes
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": 4 * n, "copy_probe_bytes_written": 4 * n}), flush=True)
        return
    from granulelayer_amd import FusedAdamW, SparsePoolingLayer
    from granulelayer_amd._native import KernelTrace

    N, K, D, B, pool = CFG["N"], CFG["K"], CFG["D"], CFG["B"], CFG["pool"]
    G = N // pool
    dev = torch.device("cuda", 0)
    t0 = time.time()
    log(f"building layer N={N:,} K={K} D={D} G={G:,} on {torch.cuda.get_device_name(0)}")
    pooling = POOLINGS[args.pooling][0]
    lay = SparsePoolingLayer(D, N, G, fan_in=K, shared_neurons=None, pooling=pooling, dtype=torch.float32, plan=_plan(),
                             device=dev, seed=0)
    lay.enable_main_grad()
    opt = FusedAdamW(lay.parameters(), lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, moments="fp32")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    x = torch.randn(B, D, generator=gen, device=dev)
    dy = torch.randn(B, G, generator=gen, device=dev)
    torch.cuda.synchronize()
    log(f"layer ready in {time.time() - t0:.1f} s")
    setup = setup_times(lay, x)
    log(f"layer setup (gather schedule, windows, edge list): {setup}")

    def step():
        y = lay(x)
        y.backward(dy)
        opt.step()

    for i in range(args.warmup):
        step()
        torch.cuda.synchronize()
        log(f"warmup step {i + 1}/{args.warmup} done")
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with KernelTrace(max_launches=128 * args.steps) as tr:
        ev0.record()
        w0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        ev1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - w0
    ms_step = ev0.elapsed_time(ev1) / args.steps
    ktimes = tr.times_ms()
    log(f"timed {args.steps} steps: {ms_step:.3f} ms/step (wall {wall / args.steps * 1e3:.3f} ms)")
    # the same step with the other relu_bits mode, for comparison (same layer, same inputs)
    other = "recompute" if RELU_BITS == "keep" else "keep"
    lay.plan.relu_bits = other
    for _ in range(2):
        step()
    torch.cuda.synchronize()
    with KernelTrace(max_launches=128 * args.steps) as tr2:
        ev0.record()
        for _ in range(args.steps):
            step()
        ev1.record()
        torch.cuda.synchronize()
    other_ms = ev0.elapsed_time(ev1) / args.steps
    other_k = {k: round(sum(v) / len(v), 4) for k, v in tr2.times_ms().items()}
    lay.plan.relu_bits = RELU_BITS
    log(f"relu_bits={other}: {other_ms:.3f} ms/step")

    # forward only (BASELINE C2 headline), same layer
    with torch.no_grad():
        for _ in range(2):
            lay(x)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            lay(x)
        e1.record()
        torch.cuda.synchronize()
    fwd_ms = e0.elapsed_time(e1) / args.steps
    log(f"forward only: {fwd_ms:.3f} ms")
    del lay, opt, x, dy
    torch.cuda.empty_cache()

    E = N * K
    kernels = {}
    for name, ts in ktimes.items():
        step_ms = sum(ts) / args.steps  # all launches of the kernel in one step
        by, fl = algorithmic(name, B, N, K, D, G, relu_bits=RELU_BITS == "keep")
        rec = {"ms": round(sum(ts) / len(ts), 4), "launches_per_step": len(ts) // args.steps,
               "ms_per_step": round(step_ms, 4)}
        if by is not None:
            rec["alg_GBps"] = round(by / (step_ms * 1e-3) / 1e9, 1)
            rec["hbm_frac"] = round(by / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
            rec["fp32_frac"] = round(fl / (step_ms * 1e-3) / 1e12 / FP32_PEAK_TFLOPS, 4)
        kernels[name] = rec
    dom = max(ktimes, key=lambda n: sum(ktimes[n]))
    dom_ms = sum(ktimes[dom]) / args.steps
    dom_launch_ms = sum(ktimes[dom]) / len(ktimes[dom])
    by, fl = algorithmic(dom, B, N, K, D, G, relu_bits=RELU_BITS == "keep")
    prof = read_profile(os.path.join(ROOT, "profiles", "pmc_c2_train_step.txt")).get(dom, {})
    if dom == "adam_kernel":
        roof = {"bound": "hbm", "achieved": round(by / (dom_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s"}
    else:
        # fp32 FMA on the vector ALUs: a gather path, no MFMA (north star).  The peak is MI355X's
        # published fp32 figure (157.3 TFLOP/s, packed issue); code built without packed-FP32
        # instructions can issue at most half of it
        roof = {"bound": "valu", "achieved": round(fl / (dom_ms * 1e-3) / 1e12, 2), "peak": FP32_PEAK_TFLOPS,
                "unit": "TFLOP/s", "compute": "fp32 VALU FMA (no MFMA; non-packed issue limit 78.65 TFLOP/s)"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes; withheld when
    # the profiled kernel's duration is more than 10% from this run's (the kernel has changed since)
    traffic, pms = prof.get("traffic"), prof.get("profile_ms")
    fresh = traffic is not None and pms is not None and abs(pms - dom_launch_ms) <= 0.1 * dom_launch_ms
    roof["traffic"] = int(traffic) if fresh else None
    roof["traffic_profile_ms"] = pms
    roof["kernel"] = dom
    roof["ms"] = round(dom_launch_ms, 4)
    roof["algorithmic_bytes"] = by
    roof["algorithmic_flops"] = fl

    value = B * E / (ms_step * 1e-3) / 1e9
    out = {
        "metric": "train-step ms & G edge-MAC/s at 100M neurons fan-in 8, B=256; % of HBM peak",
        "value": round(value, 2),
        "unit": "G edge-MAC/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded: uniform distinct indices, W~N(0,1/8), bias 0, X and dY ~N(0,1))",
        "config": {"workload": "C2-shaped train step: fwd + recompute bwd (dX, dW, db) + fused AdamW",
                   "neurons": N, "fan_in": K, "d_in": D, "batch": B, "pool": pool, "groups": G,
                   "pooling": POOLINGS[args.pooling][1], "x_dtype": "f32", "moments": "f32",
                   "relu_bits": RELU_BITS, "parallelism": "single GPU"},
        "other_relu_bits": {"relu_bits": other, "ms_per_step": round(other_ms, 3),
                            "G_edge_macs_per_s": round(B * E / (other_ms * 1e-3) / 1e9, 2), "kernels_ms": other_k},
        "fwd_ms": round(fwd_ms, 3),
        "fwd_G_edge_macs_per_s": round(B * E / (fwd_ms * 1e-3) / 1e9, 2),
        "setup": setup,
        "kernels": kernels,
        "roofline": roof,
    }
    pr1, first = None, None
    if not args.no_extra or not args.no_cpu_baseline:
        pr1 = c1_problem()
        c1_ms, first = c1_gpu(pr1, max(args.steps, 20), 3)
        out["c1_gpu"] = {"workload": "BASELINE configs[0] (C1) train step on the GPU: B=64, D=1024, N=1,048,576, "
                                     "fan-in 8, pools of 256, fp32",
                         "ms_per_step": round(c1_ms, 4),
                         "G_edge_macs_per_s": round(pr1.B * pr1.edges / (c1_ms * 1e-3) / 1e9, 2)}
        log(f"C1 on the GPU: {c1_ms:.3f} ms/step")
    if not args.no_extra:
        log("C4 full training step")
        out["c4"] = c4_step(3, 1)
        log(f"C4: {out['c4']['ms_per_step']} ms/step")
    if not args.no_cpu_baseline:
        log(f"cpu baseline: C1 x {args.cpu_steps} steps")
        out["cpu_baseline"] = cpu_baseline(pr1, args.cpu_steps, first)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
