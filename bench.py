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

Usage: python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--no-cpu-baseline]
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


def algorithmic(kernel: str, B: int, N: int, K: int, D: int, G: int, x_bytes: int = 4):
    """(bytes, flops) of one training step's launches of a kernel (one launch each, except the
    AdamW kernel: one launch for the weights, one for the bias): every input read once, every
    output written once."""
    E = N * K
    if kernel == "fwd_kernel":
        # idx + W + bias, X once, pooled output
        return 4 * E + 4 * E + 4 * N + B * D * x_bytes + 4 * B * G, 2 * B * E
    if kernel == "bwd_w_kernel":
        # idx + W + bias, X once, dW/db read-modify-write, mask bits written
        return 4 * E + 4 * E + 4 * N + B * D * x_bytes + 8 * E + 8 * N + N * B // 8, 4 * B * E
    if kernel == "dx_kernel":
        # per edge: record, weight and the neuron's B mask bits; dX written once
        return E * (4 + 4 + B // 8) + 4 * B * D, 2 * B * E
    if kernel == "adam_kernel":
        return 32 * (E + N), 12 * (E + N)
    return None, None


def read_traffic(path: str) -> dict:
    """Calibrated HBM bytes per launch of each kernel from a committed rocprofv3 summary: lines
    ``traffic <kernel> <bytes>`` (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by what the
    counter reads for a device copy of known size)."""
    out = {}
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic":
                    out[parts[1]] = int(float(parts[2]))
    except OSError:
        pass
    return out


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
    with KernelTrace(max_launches=32 * steps) as tr:
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


def cpu_baseline(groups: int, steps: int):
    import torch

    from granulelayer_amd.synthetic import make_problem
    from oracle.reference_port import PortStep

    pr = make_problem("C2", device="cpu", seed=0, groups=groups)
    st = PortStep(pr.idx, pr.w, pr.b, pr.layout.counts_tensor("cpu"), pr.layout.slots_per_group, pool="sum")
    x = pr.x.float()
    st.step(x, pr.dy)  # warm-up
    times = [st.step(x, pr.dy)["step"] for _ in range(steps)]
    t = sorted(times)[len(times) // 2]
    macs = pr.B * pr.edges
    return {"value": round(macs / t / 1e9, 4), "unit": "G edge-MAC/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"C2 train step (fwd+bwd+torch.optim.Adam) on {groups} of 98,304 pools "
                       f"({groups * 1024:,} neurons, B=256, D=4096), materialising torch restatement of "
                       f"sparse_pooling/reference on the host; median of {steps} steps = {t * 1e3:.1f} ms; "
                       f"cpu: {cpu_model()}, os.cpu_count()={os.cpu_count()}")}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-groups", type=int, default=768, help="pools in the CPU baseline's sample")
    ap.add_argument("--cpu-steps", type=int, default=5)
    ap.add_argument("--config", choices=sorted(CONFIG_WORK), default=None,
                    help="time one BASELINE config's own work at full size instead of the headline step")
    ap.add_argument("--pooling", choices=("sum", "mean", "max", "topk"), default="sum",
                    help="pooling of the train-step layer (default: the headline's sum of relu; max: the "
                         "reference's defaults, relu(max z), winners saved for backward; topk: top-8 mean, "
                         "slots saved)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (calibrates rocprofv3 byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build measures one MI355X (--gpus {args.gpus} requested); "
              "multi-GPU sharding is described in DESIGN.md but not implemented", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    if args.config:
        run_config(args.config, args.steps, args.warmup)
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
    pooling = {"type": "topk_mean", "k": 8} if args.pooling == "topk" else args.pooling
    lay = SparsePoolingLayer(D, N, G, fan_in=K, shared_neurons=None, pooling=pooling, dtype=torch.float32,
                             device=dev, seed=0)
    lay.enable_main_grad()
    opt = FusedAdamW(lay.parameters(), lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, moments="fp32")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    x = torch.randn(B, D, generator=gen, device=dev)
    dy = torch.randn(B, G, generator=gen, device=dev)
    torch.cuda.synchronize()
    log(f"layer ready in {time.time() - t0:.1f} s")

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
    with KernelTrace(max_launches=32 * args.steps) as tr:
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

    E = N * K
    kernels = {}
    for name, ts in ktimes.items():
        step_ms = sum(ts) / args.steps  # all launches of the kernel in one step
        by, fl = algorithmic(name, B, N, K, D, G)
        rec = {"ms": round(sum(ts) / len(ts), 4), "launches_per_step": len(ts) // args.steps,
               "ms_per_step": round(step_ms, 4)}
        if by is not None:
            rec["alg_GBps"] = round(by / (step_ms * 1e-3) / 1e9, 1)
            rec["hbm_frac"] = round(by / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
            rec["fp32_frac"] = round(fl / (step_ms * 1e-3) / 1e12 / FP32_PEAK_TFLOPS, 4)
        kernels[name] = rec
    dom = max(ktimes, key=lambda n: sum(ktimes[n]))
    dom_ms = sum(ktimes[dom]) / args.steps
    by, fl = algorithmic(dom, B, N, K, D, G)
    traffic = read_traffic(os.path.join(ROOT, "profiles", "pmc_c2_train_step.txt")).get(dom)
    if dom == "adam_kernel":
        roof = {"bound": "hbm", "achieved": round(by / (dom_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s"}
    else:
        # fp32 arithmetic on the vector ALUs (no MFMA on this gather path): the fp32 peak is the
        # figure MI355X publishes for fp32 (157.3 TFLOP/s, packed issue); code built without
        # packed-FP32 instructions can issue at most half of it
        roof = {"bound": "mfma", "achieved": round(fl / (dom_ms * 1e-3) / 1e12, 2), "peak": FP32_PEAK_TFLOPS,
                "unit": "TFLOP/s", "compute": "fp32 VALU FMA (no MFMA; non-packed issue limit 78.65 TFLOP/s)"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    roof["traffic"] = traffic
    roof["kernel"] = dom
    roof["ms"] = round(dom_ms, 4)
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
                   "pooling": {"sum": "sum(relu)", "mean": "mean(relu)", "max": "relu(max z)",
                               "topk": "top-8 mean(z)"}[args.pooling], "x_dtype": "f32", "moments": "f32", "parallelism": "single GPU"},
        "fwd_ms": round(fwd_ms, 3),
        "fwd_G_edge_macs_per_s": round(B * E / (fwd_ms * 1e-3) / 1e9, 2),
        "kernels": kernels,
        "roofline": roof,
    }
    if not args.no_cpu_baseline:
        log(f"cpu baseline: {args.cpu_groups} pools x {args.cpu_steps} steps")
        out["cpu_baseline"] = cpu_baseline(args.cpu_groups, args.cpu_steps)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
