"""Benchmark of the batched predictive-coding relaxation on one MI355X.

A bench "step" is one pass of the hot path over one batch: settling B samples
for T relaxation steps (BatchedPcForward.InferGetTopBatch), inputs and weights
already resident in HBM.  The metric is relaxed sample-steps per second,
value = B * T * K / elapsed over K timed passes.

Workloads:
  c1  784-256-256-10 tanh fp32, B=64, T=20, eta=0.1, x0~U[0,1]
  c2  1024-1024-1024-1024-256 tanh fp32, B=1024, T=50, eta=0.05, x0~N(0,1)   (default)
  c3  6 x 4096 GELU bf16 operands, B=4096, T=32, eta=0.05, W~N(0,1/fan_in)
  c5  12 x 8192 GELU bf16 operands, B=8192, T=16, eta=0.02, W~N(0,1/fan_in)
(c4, the ragged early-exit workload, is timed by --config c4 through the
ragged entry point.)

The JSON line carries the roofline of the dominant kernel (average duration
of its launches from HIP events on the library's stream) and a CPU baseline:
the repo's CPU restatement of the reference path timed on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {"f32": 157.3e12, "bf16": 2.5e15, "f16": 2.5e15}   # dense MFMA, MI355X
HBM_PEAK = 8.0e12

CONFIGS = {
    "c1": dict(sizes=[784, 256, 256, 10], act=1, dtype="f32", batch=64, T=20, eta=0.1, x="uniform01", init="xavier"),
    "c2": dict(sizes=[1024, 1024, 1024, 1024, 256], act=1, dtype="f32", batch=1024, T=50, eta=0.05, x="normal",
               init="xavier"),
    "c3": dict(sizes=[4096] * 6, act=4, dtype="bf16", batch=4096, T=32, eta=0.05, x="normal", init="fanin"),
    "c5": dict(sizes=[8192] * 12, act=4, dtype="bf16", batch=8192, T=16, eta=0.02, x="normal", init="fanin"),
}
ACT_NAME = {1: "tanh", 4: "gelu"}


def flops_per_sample_step(sizes):
    return 4.0 * sum(sizes[l] * sizes[l - 1] for l in range(1, len(sizes)))


def make_weights(cfg, seed=0):
    """Synthetic weights from a seeded generator (torch on the GPU for speed)."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    W, b = [], []
    s = cfg["sizes"]
    for l in range(1, len(s)):
        std = np.sqrt(2.0 / (s[l] + s[l - 1])) if cfg["init"] == "xavier" else np.sqrt(1.0 / s[l])
        w = torch.randn((s[l - 1], s[l]), generator=g, device="cuda", dtype=torch.float32) * float(std)
        W.append(w.cpu().numpy())
        b.append(np.zeros(s[l - 1], np.float32))
    return W, b


def make_inputs(cfg, seed=1):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    shape = (cfg["batch"], cfg["sizes"][0])
    if cfg["x"] == "uniform01":
        return torch.rand(shape, generator=g, device="cuda", dtype=torch.float32)
    return torch.randn(shape, generator=g, device="cuda", dtype=torch.float32)


def cpu_baseline(cfg, W, b, x_host, budget_s=10.0):
    """The oracle's restatement of BatchedPcForward + CpuGemmProvider on the
    host cores, on a bounded sample: `rows` samples for `steps` steps."""
    from oracle import pc_oracle
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
    pc_oracle.set_threads(threads)
    sizes, act = cfg["sizes"], ACT_NAME[cfg["act"]]
    P = [1.0] * len(sizes)
    # calibrate on one step of a small slice, then size the sample to the budget
    rows = min(cfg["batch"], max(4 * threads, 16))
    t0 = time.perf_counter()
    pc_oracle.batched_relax(sizes, act, cfg["eta"], W, b, P, x_host[:rows], 1)
    per = (time.perf_counter() - t0) / rows
    steps = int(max(1, min(cfg["T"], budget_s / max(per * rows, 1e-9))))
    if steps == cfg["T"]:
        rows = int(max(rows, min(cfg["batch"], budget_s / max(per * cfg["T"], 1e-9))))
        rows = min(rows, cfg["batch"])
    t0 = time.perf_counter()
    pc_oracle.batched_relax(sizes, act, cfg["eta"], W, b, P, x_host[:rows], steps)
    dt = time.perf_counter() - t0
    return {"value": rows * steps / dt, "unit": "sample-steps/s", "cores": threads, "kind": "port",
            "sample": f"oracle batched fp32 relaxation (i-k-j row-parallel GEMM as Gemm.cs:106-124), "
                      f"{rows} of {cfg['batch']} samples x {steps} of {cfg['T']} steps, {dt:.1f} s"}


def traffic_from_profiles(workload):
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--tile", type=int, default=0, help="force the GEMM tile rows (and columns unless --tile-n)")
    ap.add_argument("--tile-n", type=int, default=0)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build runs the relaxation on a single MI355X "
              "(the batch shards over GPUs with no per-step communication; see DESIGN.md).", file=sys.stderr)
        sys.exit(2)

    import torch
    from predicitivecoding_amd import GenerativeSnapshot, PcDeviceModel

    cfg = CONFIGS[args.config]
    sizes, B, T = cfg["sizes"], cfg["batch"], cfg["T"]
    print(f"# bench {args.config}: sizes={sizes} B={B} T={T} dtype={cfg['dtype']}", file=sys.stderr, flush=True)
    W, b = make_weights(cfg)
    snap = GenerativeSnapshot(sizes, cfg["act"], cfg["eta"], 0.0, False, W, b, [1.0] * len(sizes))
    model = PcDeviceModel(snap, cfg["dtype"])
    if args.tile:
        model.set_option("tile", args.tile)
        if args.tile_n:
            model.set_option("tile_n", args.tile_n)
    x = make_inputs(cfg)
    top = torch.empty((B, sizes[-1]), device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()

    def one_pass():
        model.relax_device(x.data_ptr(), B, T, top.data_ptr())

    for _ in range(args.warmup):
        one_pass()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_pass()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    value = B * T * args.steps / elapsed
    print(f"# timed {args.steps} passes: {ms_per_step:.3f} ms/pass, {value:.4g} sample-steps/s",
          file=sys.stderr, flush=True)

    # Roofline: the same passes again with HIP events around every phase launch
    # (eager launches on the library's stream), averaged per phase.
    model.set_option("profile", 1)
    err_ms = upd_ms = 0.0
    launches = 0
    for _ in range(max(1, min(args.steps, 5))):
        one_pass()
        e, u, n = model.profile_result()
        err_ms += e * n
        upd_ms += u * n
        launches += n
    torch.cuda.synchronize()
    model.set_option("profile", 0)
    err_ms /= launches
    upd_ms /= launches
    dom_name, dom_ms = ("update_phase", upd_ms) if upd_ms >= err_ms else ("error_phase", err_ms)
    flop_launch = 2.0 * B * sum(sizes[l] * sizes[l - 1] for l in range(1, len(sizes)))
    achieved = flop_launch / (dom_ms * 1e-3)
    peak = PEAK[cfg["dtype"]]
    roofline = {"bound": "mfma", "achieved": achieved / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s",
                "frac": achieved / peak, "traffic": traffic_from_profiles(args.config),
                "kernel": dom_name, "kernel_ms": dom_ms, "error_phase_ms": err_ms, "update_phase_ms": upd_ms,
                "flop_per_launch": flop_launch, "launches_timed": launches,
                "path_frac": (flops_per_sample_step(sizes) * value) / peak}
    print(f"# roofline: error {err_ms:.4f} ms, update {upd_ms:.4f} ms per launch; {dom_name} at "
          f"{achieved / 1e12:.1f} TFLOP/s = {100 * achieved / peak:.1f}% of peak", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        x_host = x.cpu().numpy()
        cpu = cpu_baseline(cfg, W, b, x_host, args.cpu_budget)
        print(f"# cpu baseline: {cpu['value']:.4g} sample-steps/s on {cpu['cores']} threads", file=sys.stderr,
              flush=True)

    rec = {
        "metric": "relaxed samples*steps/sec at 1 GPU and % of MFMA/HBM roofline",
        "value": value,
        "unit": "sample-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded random weights and inputs)",
        "config": {"workload": f"{args.config}: {'-'.join(map(str, sizes))} {ACT_NAME[cfg['act']]} "
                               f"{cfg['dtype']}, B={B}, T={T}, eta={cfg['eta']}",
                   "batch": B, "relax_steps": T, "layer_sizes": sizes, "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec))
    model.close()


if __name__ == "__main__":
    main()
