"""Benchmark of the batched predictive-coding relaxation on one MI355X.

A bench "step" is one pass of the hot path over one batch: settling B samples
for T relaxation steps (BatchedPcForward.InferGetTopBatch), inputs and weights
already resident in HBM.  The metric is relaxed sample-steps per second,
value = B * T * K / elapsed over K timed passes.

Workloads:
  c1  784-256-256-10 tanh fp32, B=64, T=20, eta=0.1, x0~U[0,1]
  c2  1024-1024-1024-1024-256 tanh fp32, B=1024, T=50, eta=0.05, x0~N(0,1)
  c3  6 x 4096 GELU bf16 operands, B=4096, T=32, eta=0.05, W~N(0,1/fan_in)
      (the configuration the bf16 MFMA target is stated on)
  c5  12 x 8192 GELU bf16 operands, B=8192, T=16, eta=0.02, W~N(0,1/fan_in)
      (default: the largest configuration of the five, which one GPU holds)
  c4  ragged: 64 requests on a shared 4 x 2048 tanh fp32 network, per-request
      batch log-uniform in [1,512] and T uniform in [8,64] (seeded), early exit
      when energy/sample < 1e-3; one pass = one packed pcd_pc_relax_ragged call,
      value = sum over requests of rows x steps actually run / elapsed.
  c4x c4's requests under the relative exit rule (Network.SettleAdaptive) at
      epsilon 1e-2, at which most requests leave before their budget.
  c1cls    c1's network classifying a batch of 64 by minimum energy
           (Network.PredictCore per sample: 10 settlings with the top clamped
           to each one-hot label); value counts the 640 settled rows x T.
  c1learn  c1's network taking a learning step (Network.Learn) on a batch of
           64 labelled samples; value counts 64 rows x T.
  gemm     the GEMM provider (pcd_gemm_bf16) on 8192^3, in TFLOP/s.
  pub      the reference's own published workload (MixedPrecisionBench):
           [3072,512,128,10] tanh, eta 0.05, 64 inputs, T=20, host arrays in
           and out through the drop-in, median of repeated calls, beside the
           published RTX 4070 SUPER / Ryzen figures.

The default line (c5) also carries, under "extra", the c3 record (the
configuration the bf16 target is stated on) and the pub record, and under
"pcie_inclusive" the c5 pass with its input and output on the host.

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
    # eta and the initialisation are unstated for c4: NetworkConfig's default state rate (0.1) and
    # Xavier-normal, the reference's tanh initialiser
    "c4": dict(sizes=[2048] * 4, act=1, dtype="f32", eta=0.1, x="normal", init="xavier", requests=64,
               bmax=512, tmin=8, tmax=64, exit_rule="absolute", exit_thr=1e-3, seed=4),
    # c4's requests under the reference's relative exit rule (Network.SettleAdaptive, Network.cs:876-907):
    # requests leave at data-dependent steps, which c4's own absolute rule never makes them do.  Not one of
    # the reference's five configs; epsilon 1e-2 (the effort presets' 1e-3..1e-5 never fire within 64 steps).
    "c4x": dict(sizes=[2048] * 4, act=1, dtype="f32", eta=0.1, x="normal", init="xavier", requests=64,
                bmax=512, tmin=8, tmax=64, exit_rule="relative", exit_thr=1e-2, seed=4),
    # c1's network used the way the reference's Trainer does: minimum-energy
    # classification of a batch (Network.PredictCore per sample, 10 clamped
    # settlings each) and the learning step (Network.Learn) on a batch
    "c1cls": dict(sizes=[784, 256, 256, 10], act=1, dtype="f32", batch=64, T=20, eta=0.1, x="uniform01",
                  init="xavier", mode="classify"),
    "c1learn": dict(sizes=[784, 256, 256, 10], act=1, dtype="f32", batch=64, T=20, eta=0.1, x="uniform01",
                    init="xavier", mode="learn", eta_w=0.01),
    # c5's network at a serving batch of 64 rows: both weight copies (W and W^T,
    # 1.48 GB each in bf16, far beyond the 256 MB MALL) stream from HBM in every
    # phase, at about 64 FLOP/B, below the bf16 ridge of 312: the small-batch
    # variant on which the HBM-bandwidth target means something.  Not one of
    # the reference's five configs.
    "c5s": dict(sizes=[8192] * 12, act=4, dtype="bf16", batch=64, T=16, eta=0.02, x="normal", init="fanin"),
    # the GEMM provider slot (IGemmProvider / CudaGemmProvider.MatMulDeviceExBf16) on c5's layer shape
    "gemm": dict(dtype="bf16", m=8192, k=8192, n=8192),
    # the reference's own published batched-forward workload (tools/MixedPrecisionBench/Program.cs:75-127):
    # [3072,512,128,10] tanh, StateLearningRate 0.05, 64 inputs ~N(0,1), 20 steps, host arrays in and out;
    # published (ROADMAP-MixedPrecision.md:99, Ryzen-class CPU + RTX 4070 SUPER): per-sample loop 574 ms,
    # batched CPU 158 ms, batched CUDA float 75 ms, CUDA mixed (fp16) 94 ms per call
    "pub": dict(sizes=[3072, 512, 128, 10], act=1, dtype="f32", batch=64, T=20, eta=0.05, x="normal",
                init="xavier", published_ms={"per_sample_loop": 574.0, "cpu_batched": 158.0, "cuda_float": 75.0,
                                             "cuda_mixed": 94.0}),
}
ACT_NAME = {1: "tanh", 4: "gelu"}


def apply_options(model, args):
    for item in args.option:
        name, _, value = item.partition("=")
        model.set_option(name, int(value))


def flops_per_sample_step(sizes):
    return 4.0 * sum(sizes[l] * sizes[l - 1] for l in range(1, len(sizes)))


def phase_bytes(sizes, B, dtype):
    """Algorithmic HBM bytes of one error-phase and one update-phase launch:
    every operand read and every result written once.  Error phase, per layer
    l: W_l, the state operand S_l, M_{l-1} read and X_{l-1} written (fp32), D
    written (operand type), and for l >= 2 the fp32 state M_{l-1} again for the
    folded X.  Update phase: W_l^T, D_l, X_l read and M_l written (fp32), plus
    the 16-bit copy S_l."""
    wb = 4 if dtype == "f32" else 2
    ab = wb
    err = upd = 0
    for l in range(1, len(sizes)):
        s_l, s_p = sizes[l], sizes[l - 1]
        err += s_l * s_p * wb + B * s_l * ab + B * s_p * (4 + ab) + (4 * B * s_p if l >= 2 else 0)
        upd += s_l * s_p * wb + B * s_p * ab + 8 * B * s_l + (2 * B * s_l if wb == 2 else 0)
    return float(err), float(upd)


MALL_BYTES = 256 << 20   # MI355X Infinity Cache


def topology(sizes):
    """Layer widths as "8192x12" when every layer has one width, else "784-256-256-10"."""
    if len(set(sizes)) == 1:
        return f"{sizes[0]}×{len(sizes)}"
    return "-".join(map(str, sizes))


def working_set_bytes(sizes, B, dtype):
    """Device bytes a settling step touches: W and W^T in the operand type, and
    the fp32 states M, X, the operand copies S, D of the batch."""
    wb = 4 if dtype == "f32" else 2
    w = sum(2 * sizes[l] * sizes[l - 1] * wb for l in range(1, len(sizes)))
    st = sum(B * s * (4 + 4 + (wb if wb == 2 else 0)) for s in sizes) + \
        sum(B * sizes[l - 1] * wb for l in range(1, len(sizes)))
    return float(w + st)


def traffic_fields(sizes, B, dtype):
    """What the counter-derived `traffic` figure counts, for this working set:
    FETCH_SIZE and WRITE_SIZE count L2 fills and write-backs; when the whole
    working set fits the 256 MB MALL, those fills are mostly served by the
    MALL, so the figure is L2-miss traffic, an upper bound on HBM traffic."""
    ws = working_set_bytes(sizes, B, dtype)
    return {"traffic_counts": "L2 fills (FETCH_SIZE) + L2 write-backs (WRITE_SIZE), per launch, copy-calibrated",
            "working_set_bytes": ws, "mall_resident": ws <= MALL_BYTES}


def make_ragged_requests(cfg):
    """Per-request rows (log-uniform in [1, bmax]) and step budgets (uniform in
    [tmin, tmax]) from the config's seed."""
    rng = np.random.default_rng(cfg["seed"])
    rows = np.floor(np.exp(rng.uniform(0.0, np.log(cfg["bmax"]), cfg["requests"]))).astype(np.int64)
    rows = np.clip(rows, 1, cfg["bmax"]).astype(np.int32)
    steps = rng.integers(cfg["tmin"], cfg["tmax"] + 1, cfg["requests"]).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(rows)]).astype(np.int32)
    return offsets, steps


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


CPU_REPS = 3


def host_nproc():
    """Host cores this process may run on (what `nproc` prints)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_threads():
    """Threads of the CPU baseline: every core `nproc` reports, unless
    OMP_NUM_THREADS names the share of the host this process was given."""
    return int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or host_nproc()


def cpu_model():
    """The host CPU's model name (from /proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def host_fields(threads):
    """CPU facts the baseline record carries beside its thread count."""
    return {"nproc": host_nproc(), "cpu_model": cpu_model(),
            "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"), "threads": threads}


def median_run(run, reps=CPU_REPS):
    """Times `run` (after the caller's warm-up call) `reps` times; returns
    (median seconds, the run's result), as the reference's bench harness
    reports MedianMs(reps: 3, warmup: 1) (tools/MixedPrecisionBench/Program.cs:96-101)."""
    times, out = [], None
    for _ in range(reps):
        t0 = time.perf_counter()
        out = run()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), out


def cpu_baseline(cfg, W, b, x_host, budget_s=10.0):
    """The oracle's restatement of BatchedPcForward + CpuGemmProvider on the
    host cores, on a bounded sample: `rows` samples for `steps` steps, the
    median of three runs."""
    from oracle import pc_oracle
    threads = cpu_threads()
    pc_oracle.set_threads(threads)
    sizes, act = cfg["sizes"], ACT_NAME[cfg["act"]]
    P = [1.0] * len(sizes)
    # calibrate on one step of a small slice (after one untimed call that
    # starts the thread pool and warms the caches), then size the sample to
    # the budget
    rows = min(cfg["batch"], max(4 * threads, 16))
    pc_oracle.batched_relax(sizes, act, cfg["eta"], W, b, P, x_host[:rows], 1)
    t0 = time.perf_counter()
    pc_oracle.batched_relax(sizes, act, cfg["eta"], W, b, P, x_host[:rows], 2)
    per = (time.perf_counter() - t0) / (2 * rows)
    run_s = budget_s / CPU_REPS
    steps = int(max(1, min(cfg["T"], run_s / max(per * rows, 1e-9))))
    if steps == cfg["T"]:
        rows = int(max(rows, min(cfg["batch"], run_s / max(per * cfg["T"], 1e-9))))
        rows = min(rows, cfg["batch"])
    print(f"# cpu baseline sample: {rows} rows x {steps} steps (calibrated {per * 1e3:.3f} ms per "
          f"sample-step), median of {CPU_REPS}", file=sys.stderr, flush=True)
    dt, _ = median_run(lambda: pc_oracle.batched_relax(sizes, act, cfg["eta"], W, b, P, x_host[:rows], steps))
    return {"value": rows * steps / dt, "unit": "sample-steps/s", "cores": threads, **host_fields(threads), "kind": "port",
            "sample": f"oracle batched fp32 relaxation (i-k-j row-parallel GEMM as Gemm.cs:106-124), "
                      f"{rows} of {cfg['batch']} samples x {steps} of {cfg['T']} steps, median of {CPU_REPS} "
                      f"runs of {dt:.1f} s"}


def traffic_from_profiles(workload, kernel):
    """HBM bytes per launch of `kernel` ("error_phase", "update_phase", "plain") from
    the committed PMC summary profiles/traffic_<workload>.json (written by
    --traffic-from), or None when it has not been measured."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f)["kernels"][kernel]["bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None


COPY_CALIB_BYTES = 1 << 30


def calibrate_copy():
    """One elementwise copy of COPY_CALIB_BYTES (torch.mul by 1 into a new
    tensor: reads and writes exactly that many bytes).  Profiled with
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, it gives the factor between the
    counters and real bytes."""
    import torch
    x = torch.ones(COPY_CALIB_BYTES // 4, device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()
    y = torch.mul(x, 1.0)
    torch.cuda.synchronize()
    print(f"# copy calibration: {COPY_CALIB_BYTES} bytes read and written ({float(y[0])})", file=sys.stderr)


def _pmc_rows(directory):
    """Rows of every rocprofv3 counter_collection.csv under `directory`."""
    import csv
    import glob
    rows = []
    for path in glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            rows.extend(csv.DictReader(f))
    if not rows:
        raise SystemExit(f"no counter_collection.csv under {directory}")
    return rows


def _mean_counter(rows, counter, name_filter):
    """Mean per dispatch of `counter` over the dispatches whose kernel name
    passes name_filter (a counter's per-dispatch value is the sum of its
    instance rows)."""
    per_dispatch = {}
    for r in rows:
        if r.get("Counter_Name") != counter or not name_filter(r.get("Kernel_Name", "")):
            continue
        key = r.get("Dispatch_Id") or r.get("Correlation_Id")
        per_dispatch[key] = per_dispatch.get(key, 0.0) + float(r["Counter_Value"])
    if not per_dispatch:
        return None, 0
    return sum(per_dispatch.values()) / len(per_dispatch), len(per_dispatch)


def traffic_from_pmc(workload, fetch_dir, write_dir, calib_fetch_dir, calib_write_dir, command, out_path=None):
    """Writes profiles/traffic_<workload>.json (or out_path): HBM bytes per
    launch of each phase kernel from FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch), each scaled by what the same counter reads for the calibration
    copy."""
    is_copy = lambda n: "MulFunctor" in n
    cf, _ = _mean_counter(_pmc_rows(calib_fetch_dir), "FETCH_SIZE", is_copy)
    cw, _ = _mean_counter(_pmc_rows(calib_write_dir), "WRITE_SIZE", is_copy)
    if cf is None or cw is None:
        raise SystemExit("no calibration copy dispatches in the calibration runs")
    f_fetch = cf * 1024.0 / COPY_CALIB_BYTES
    f_write = cw * 1024.0 / COPY_CALIB_BYTES
    fr, wr = _pmc_rows(fetch_dir), _pmc_rows(write_dir)
    out = {"workload": workload, "command": command,
           "calibration": {"bytes": COPY_CALIB_BYTES, "fetch_kib": cf, "write_kib": cw,
                           "fetch_factor": f_fetch, "write_factor": f_write},
           "kernels": {}}
    import re
    # phase_kernel<OP, BM, BN, EPI> or phase_kernel<OP, BM, BN, EPI, direct-weight flag>
    epi_of = re.compile(r"phase_kernel<[^,<>]+, \d+, \d+, (\d)(?:, (?:true|false))?>\(pcd::ProblemSet, pcd::PhaseArgs\)")
    for name, epi in (("error_phase", "0"), ("update_phase", "1"), ("plain", "3")):
        def sel(n, epi=epi):
            m = epi_of.search(n)
            return m is not None and m.group(1) == epi
        fk, nf = _mean_counter(fr, "FETCH_SIZE", sel)
        wk, nw = _mean_counter(wr, "WRITE_SIZE", sel)
        if fk is None or wk is None:
            continue  # this workload launches no such kernel
        fetch_b = fk * 1024.0 / f_fetch
        write_b = wk * 1024.0 / f_write
        out["kernels"][name] = {"fetch_kib": fk, "write_kib": wk, "dispatches": [nf, nw],
                                "fetch_bytes": fetch_b, "write_bytes": write_b,
                                "bytes_per_launch": fetch_b + write_b}
    path = out_path or os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))

def bench_ragged(args, cfg):
    """c4, c4x: one pass = one packed pcd_pc_relax_ragged call over every request."""
    import torch
    from predicitivecoding_amd import GenerativeSnapshot, PcDeviceModel
    sizes = cfg["sizes"]
    offsets, steps = make_ragged_requests(cfg)
    rows, R = int(offsets[-1]), len(steps)
    print(f"# bench {args.config}: sizes={sizes} requests={R} rows={rows} steps {steps.min()}..{steps.max()} "
          f"exit {cfg['exit_rule']} < {cfg['exit_thr']}", file=sys.stderr, flush=True)
    W, b = make_weights(cfg)
    snap = GenerativeSnapshot(sizes, cfg["act"], cfg["eta"], 0.0, False, W, b, [1.0] * len(sizes))
    model = PcDeviceModel(snap, cfg["dtype"])
    apply_options(model, args)
    if args.tile_order >= 0:
        model.set_option("tile_order", args.tile_order)
    if args.tile:
        model.set_option("tile", args.tile)
        if args.tile_n:
            model.set_option("tile_n", args.tile_n)
    g = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn((rows, sizes[0]), generator=g, device="cuda", dtype=torch.float32)
    top = torch.empty((rows, sizes[-1]), device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()

    def one_pass():
        return model.relax_ragged_device(x.data_ptr(), offsets, steps, top.data_ptr(), cfg["exit_rule"],
                                         cfg["exit_thr"])

    for _ in range(args.warmup):
        one_pass()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    done = 0
    for _ in range(args.steps):
        used, _ = one_pass()
        done += int(np.sum(np.diff(offsets).astype(np.int64) * used))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    value = done / elapsed
    ms_per_step = elapsed * 1e3 / args.steps
    print(f"# timed {args.steps} passes: {ms_per_step:.3f} ms/pass, {value:.4g} sample-steps/s, "
          f"{int(np.sum(used < steps))} of {R} requests exited early", file=sys.stderr, flush=True)

    # Per-launch timing of the phases (eager, HIP events on the library's
    # stream) and the FLOPs those launches did: at step t the rows of every
    # request still running.
    model.set_option("profile", 1)
    used, _ = one_pass()
    err_ms, upd_ms, launches = model.profile_result()
    model.set_option("profile", 0)
    per_row = np.diff(offsets).astype(np.float64)
    active = np.array([per_row[used > t].sum() for t in range(int(steps.max()))])
    S = sum(sizes[l] * sizes[l - 1] for l in range(1, len(sizes)))
    flop_launch = 2.0 * S * active.mean()             # mean over the launches of one phase
    dom_name, dom_ms = ("update_phase", upd_ms) if upd_ms >= err_ms else ("error_phase", err_ms)
    achieved = flop_launch / (dom_ms * 1e-3)
    peak = PEAK[cfg["dtype"]]
    roofline = {"bound": "mfma", "achieved": achieved / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s",
                "frac": achieved / peak, "traffic": traffic_from_profiles(args.config, dom_name), "kernel": dom_name,
                "kernel_ms": dom_ms, "error_phase_ms": err_ms, "update_phase_ms": upd_ms, "launches_timed": launches,
                "flop_per_launch": flop_launch, "mean_active_rows": float(active.mean()),
                "path_frac": 4.0 * S * value / peak, **traffic_fields(sizes, rows, cfg["dtype"])}
    print(f"# roofline: error {err_ms:.4f} ms, update {upd_ms:.4f} ms per launch over {launches} steps, "
          f"{active.mean():.0f} active rows on average; {dom_name} at {achieved / 1e12:.1f} TFLOP/s = "
          f"{100 * achieved / peak:.1f}% of peak", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_ragged(cfg, W, b, x.cpu().numpy(), offsets, steps, args.cpu_budget)
        print(f"# cpu baseline: {cpu['value']:.4g} sample-steps/s on {cpu['cores']} threads", file=sys.stderr,
              flush=True)
    rec = {
        "metric": "relaxed samples*steps/sec at 1 GPU and % of MFMA/HBM roofline",
        "value": value, "unit": "sample-steps/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_per_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": cfg["dtype"], "data": "synthetic (seeded random weights, inputs and request shapes)",
        "config": {"workload": f"{args.config}: ragged, {R} requests on {'-'.join(map(str, sizes))} tanh f32, rows "
                               f"log-uniform [1,{cfg['bmax']}], T uniform [{cfg['tmin']},{cfg['tmax']}], exit "
                               + (f"E/rows < {cfg['exit_thr']}" if cfg["exit_rule"] == "absolute" else
                                  f"relative decrease < {cfg['exit_thr']} (SettleAdaptive)")
                               + f", {int(np.sum(used < steps))} of {R} exited early, eta={cfg['eta']}",
                   "requests": R, "rows": rows, "layer_sizes": sizes, "parallelism": "single GPU"},
        "roofline": roofline, "cpu_baseline": cpu,
    }
    print(json.dumps(rec))
    model.close()


def bench_clamped(args, cfg):
    """c1cls / c1learn: one pass = one pcd_pc_classify (every sample settled
    against every class) or one pcd_pc_learn over the batch."""
    import torch
    from predicitivecoding_amd import GenerativeSnapshot, PcDeviceModel
    sizes, B, T, mode = cfg["sizes"], cfg["batch"], cfg["T"], cfg["mode"]
    C = sizes[-1]
    rows = B * C if mode == "classify" else B
    print(f"# bench {args.config}: {mode} sizes={sizes} B={B} T={T} rows={rows}", file=sys.stderr, flush=True)
    W, b = make_weights(cfg)
    snap = GenerativeSnapshot(sizes, cfg["act"], cfg["eta"], 0.0, False, W, b, [1.0] * len(sizes))
    model = PcDeviceModel(snap, cfg["dtype"])
    apply_options(model, args)
    if args.tile_order >= 0:
        model.set_option("tile_order", args.tile_order)
    if args.tile:
        model.set_option("tile", args.tile)
    x = make_inputs(cfg)
    labels = torch.zeros((B, C), device="cuda", dtype=torch.float32)
    labels[torch.arange(B, device="cuda"), torch.arange(B, device="cuda") % C] = 1.0
    ce = torch.empty((B, C), device="cuda", dtype=torch.float32)
    cls = torch.empty((B,), device="cuda", dtype=torch.int32)
    be = torch.empty((B,), device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()

    def one_pass():
        if mode == "classify":
            model.classify_device(x.data_ptr(), B, T, ce.data_ptr(), cls.data_ptr(), be.data_ptr())
        else:
            model.learn_device(x.data_ptr(), labels.data_ptr(), B, T, cfg["eta_w"], 0.0, be.data_ptr())

    for _ in range(args.warmup):
        one_pass()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_pass()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    value = rows * T * args.steps / elapsed
    print(f"# timed {args.steps} passes: {ms_per_step:.3f} ms/pass, {value:.4g} sample-steps/s "
          f"({B * args.steps / elapsed:.4g} samples/s)", file=sys.stderr, flush=True)

    model.set_option("profile", 1)
    one_pass()
    torch.cuda.synchronize()
    err_ms, upd_ms, launches = model.profile_result()
    model.set_option("profile", 0)
    S = sum(sizes[l] * sizes[l - 1] for l in range(1, len(sizes)))
    S_free = S - sizes[-1] * sizes[-2]                 # the clamped top layer is never updated
    flops = {"error_phase": 2.0 * rows * S, "update_phase": 2.0 * rows * S_free}
    ms = {"error_phase": err_ms, "update_phase": upd_ms}
    dom_name = max(ms, key=ms.get)
    achieved = flops[dom_name] / (ms[dom_name] * 1e-3)
    peak = PEAK[cfg["dtype"]]
    roofline = {"bound": "mfma", "achieved": achieved / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s",
                "frac": achieved / peak, "traffic": traffic_from_profiles(args.config, dom_name), "kernel": dom_name,
                "kernel_ms": ms[dom_name], "error_phase_ms": err_ms, "update_phase_ms": upd_ms,
                "flop_per_launch": flops[dom_name], "launches_timed": launches,
                "path_frac": (2.0 * (S + S_free) * value) / peak, **traffic_fields(sizes, rows, cfg["dtype"])}
    print(f"# roofline: error {err_ms:.4f} ms, update {upd_ms:.4f} ms per launch; {dom_name} at "
          f"{achieved / 1e12:.1f} TFLOP/s = {100 * achieved / peak:.1f}% of peak", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_clamped(cfg, W, b, x.cpu().numpy(), labels.cpu().numpy(), args.cpu_budget)
        print(f"# cpu baseline: {cpu['value']:.4g} sample-steps/s on {cpu['cores']} threads", file=sys.stderr,
              flush=True)
    what = ("minimum-energy classification, every sample settled against each of the "
            f"{C} one-hot labels" if mode == "classify" else f"learning step, eta_w={cfg['eta_w']}")
    rec = {
        "metric": "relaxed samples*steps/sec at 1 GPU and % of MFMA/HBM roofline",
        "value": value, "unit": "sample-steps/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_per_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": cfg["dtype"], "data": "synthetic (seeded random weights and inputs)",
        "config": {"workload": f"{args.config}: {'-'.join(map(str, sizes))} tanh f32, B={B}, T={T}, "
                               f"eta={cfg['eta']}: {what}",
                   "batch": B, "relaxed_rows": rows, "relax_steps": T, "layer_sizes": sizes,
                   "samples_per_s": B * args.steps / elapsed, "parallelism": "single GPU"},
        "roofline": roofline, "cpu_baseline": cpu,
    }
    print(json.dumps(rec))
    model.close()


def cpu_baseline_clamped(cfg, W, b, x_host, labels_host, budget_s=10.0):
    """The oracle's per-sample PredictCore / Learn loop (one sample at a time,
    as Trainer.Evaluate / TrainEpoch call them), on the first samples of the
    batch until the budget is spent."""
    from oracle import pc_oracle
    pc_oracle.set_threads(1)
    sizes, act, T = cfg["sizes"], ACT_NAME[cfg["act"]], cfg["T"]
    P = [1.0] * len(sizes)
    C = sizes[-1]
    per_sample_rows = C if cfg["mode"] == "classify" else 1

    def one_pass():
        # samples one at a time until a third of the budget is spent; returns
        # the samples done and the seconds taken
        done, t0 = 0, time.perf_counter()
        Wc, bc = W, b
        while done < cfg["batch"] and (time.perf_counter() - t0) < budget_s / CPU_REPS:
            if cfg["mode"] == "classify":
                pc_oracle.classify(sizes, act, cfg["eta"], W, b, P, x_host[done:done + 1], T)
            else:
                Wc, bc, _ = pc_oracle.learn(sizes, act, cfg["eta"], Wc, bc, P, x_host[done:done + 1],
                                            labels_host[done:done + 1], T, cfg["eta_w"])
            done += 1
        return done, time.perf_counter() - t0

    one_pass()   # warm-up
    passes = [one_pass() for _ in range(CPU_REPS)]
    rates = sorted(d * per_sample_rows * T / t for d, t in passes)
    done, dt = passes[0]
    name = "Network.PredictCore" if cfg["mode"] == "classify" else "Network.Learn"
    return {"value": rates[len(rates) // 2], "unit": "sample-steps/s", "cores": 1, **host_fields(1), "kind": "port",
            "sample": f"oracle {name} one sample at a time (batch-1 settlings), median of {CPU_REPS} passes of "
                      f"about {done} of {cfg['batch']} samples x {per_sample_rows} settlings x {T} steps "
                      f"({dt:.1f} s each)"}


def bench_gemm(args, cfg):
    """gemm: one pass = one pcd_gemm_bf16 call, C = A B^T with both operands
    already K-contiguous in HBM (read in place)."""
    import torch
    from predicitivecoding_amd import DeviceTensor  # noqa: F401  (loads the library)
    from predicitivecoding_amd._native import call
    m, k, n = cfg["m"], cfg["k"], cfg["n"]
    print(f"# bench gemm: {cfg['dtype']} {m} x {k} x {n}", file=sys.stderr, flush=True)
    g = torch.Generator(device="cuda").manual_seed(0)
    A = torch.randn((m, k), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    B = torch.randn((n, k), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    C = torch.empty((m, n), device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()

    def one_pass():
        call("pcd_gemm_bf16", A.data_ptr(), B.data_ptr(), C.data_ptr(), m, k, n, 0, 1, 0.0, None)

    for _ in range(args.warmup):
        one_pass()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_pass()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    flop = 2.0 * m * n * k
    value = flop * args.steps / elapsed / 1e12
    ms = elapsed * 1e3 / args.steps
    # the launch itself, timed with events on the stream it runs on (the default stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        one_pass()
    e1.record()
    torch.cuda.synchronize()
    kms = e0.elapsed_time(e1) / args.steps
    achieved = flop / (kms * 1e-3)
    print(f"# timed {args.steps} GEMMs: {ms:.3f} ms each, {value:.1f} TFLOP/s; kernel {kms:.3f} ms", file=sys.stderr,
          flush=True)
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import pc_oracle
        threads = cpu_threads()
        pc_oracle.set_threads(threads)
        bt = B.float().cpu().numpy().T.copy()
        t0 = time.perf_counter()
        pc_oracle.gemm(A[:16].float().cpu().numpy(), bt, "bf16")     # calibration
        per_row = (time.perf_counter() - t0) / 16
        rows = int(min(m, max(16, args.cpu_budget / 2 / CPU_REPS / max(per_row, 1e-9))))
        a = A[:rows].float().cpu().numpy()
        dt, _ = median_run(lambda: pc_oracle.gemm(a, bt, "bf16"))
        cpu = {"value": 2.0 * rows * n * k / dt / 1e12, "unit": "TFLOP/s", "cores": threads, **host_fields(threads), "kind": "port",
               "sample": f"oracle mixed GEMM (Gemm.cs:44-60, i-k-j row-parallel), {rows} of {m} rows, median of "
                         f"{CPU_REPS} runs of {dt:.1f} s"}
        print(f"# cpu baseline: {cpu['value'] * 1e3:.2f} GFLOP/s on {threads} threads", file=sys.stderr, flush=True)
    rec = {
        "metric": "provider GEMM throughput at 1 GPU and % of MFMA roofline", "value": value, "unit": "TFLOP/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": cfg["dtype"], "data": "synthetic (seeded random operands)",
        "config": {"workload": f"gemm: pcd_gemm_bf16 {m} x {k} x {n}, B given transposed (K-contiguous)",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": achieved / 1e12, "peak": PEAK[cfg["dtype"]] / 1e12,
                     "unit": "TFLOP/s", "frac": achieved / PEAK[cfg["dtype"]],
                     "traffic": traffic_from_profiles("gemm", "plain"),
                     "kernel": "phase_kernel EPI_PLAIN", "kernel_ms": kms},
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec))


def cpu_baseline_ragged(cfg, W, b, x_host, offsets, steps, budget_s=10.0):
    """The oracle's per-request relaxation with the same exit rule, on the
    first requests that fit the time budget."""
    from oracle import pc_oracle
    threads = cpu_threads()
    pc_oracle.set_threads(threads)
    sizes, P = cfg["sizes"], [1.0] * len(cfg["sizes"])
    n = min(16, int(offsets[-1]))
    pc_oracle.batched_relax(sizes, "tanh", cfg["eta"], W, b, P, x_host[:n], 1)
    t0 = time.perf_counter()
    pc_oracle.batched_relax(sizes, "tanh", cfg["eta"], W, b, P, x_host[:n], 2)
    per = (time.perf_counter() - t0) / (2 * n)
    rows = np.diff(offsets)
    k, est = 0, 0.0
    while k < len(steps) and est + rows[k] * steps[k] * per <= budget_s / CPU_REPS:
        est += rows[k] * steps[k] * per
        k += 1
    k = max(k, 1)
    sub_off = offsets[:k + 1]
    dt, (used, _, _) = median_run(lambda: pc_oracle.ragged_relax(sizes, "tanh", cfg["eta"], W, b, P,
                                                                 x_host[:int(sub_off[-1])], sub_off, steps[:k],
                                                                 cfg["exit_rule"], cfg["exit_thr"]))
    done = int(np.sum(rows[:k].astype(np.int64) * used))
    return {"value": done / dt, "unit": "sample-steps/s", "cores": threads, **host_fields(threads), "kind": "port",
            "sample": f"oracle per-request fp32 relaxation with the same exit rule, first {k} of {len(steps)} "
                      f"requests ({int(sub_off[-1])} rows, {done} sample-steps), median of {CPU_REPS} runs of "
                      f"{dt:.1f} s"}



def median_ms_of(run, reps, warmup=1):
    """Median wall time of `run` in ms over `reps` calls after `warmup` untimed
    ones (the reference harness's MedianMs, Program.cs:96-101)."""
    for _ in range(warmup):
        run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)) * 1e3


def bench_published(args, standalone=False):
    """pub: the reference's published batched-forward workload, timed as its
    harness times it: one call of the drop-in (host arrays in and out,
    BatchedPcForward.infer_get_top_batch, float and mixed) per repetition, the
    median after a warm-up, beside the oracle's batched fp32 path (the
    reference's CpuGemmProvider route) and its per-sample loop on the host
    cores.  The reference's .NET Random streams cannot be reproduced: weights
    are seeded Xavier-normal as Network's tanh initialiser draws them, inputs
    seeded N(0, 1)."""
    import torch
    from predicitivecoding_amd import BatchedPcForward, GenerativeSnapshot, PcDeviceModel
    cfg = CONFIGS["pub"]
    sizes, B, T, eta = cfg["sizes"], cfg["batch"], cfg["T"], cfg["eta"]
    print(f"# bench pub: sizes={sizes} B={B} T={T} tanh f32, host arrays (the reference's published workload)",
          file=sys.stderr, flush=True)
    W, b = make_weights(cfg)
    rng = np.random.default_rng(4)
    inputs = [rng.standard_normal(sizes[0]).astype(np.float32) for _ in range(B)]
    snap = GenerativeSnapshot(sizes, cfg["act"], eta, 0.0, False, W, b, [1.0] * len(sizes))
    reps = max(3, args.steps)
    ms_float = median_ms_of(lambda: BatchedPcForward.infer_get_top_batch(snap, inputs, T), reps)
    ms_mixed = median_ms_of(lambda: BatchedPcForward.infer_get_top_batch(snap, inputs, T, mixed=True), reps)
    # the same settling on inputs already in HBM (the kernels alone, one pass)
    model = PcDeviceModel(snap, "f32")
    x = torch.from_numpy(np.stack(inputs)).cuda()
    top = torch.empty((B, sizes[-1]), device="cuda", dtype=torch.float32)

    def resident():
        model.relax_device(x.data_ptr(), B, T, top.data_ptr())
        torch.cuda.synchronize()

    ms_resident = median_ms_of(resident, reps)
    model.close()
    pub = cfg["published_ms"]
    print(f"# pub: drop-in float {ms_float:.3f} ms, mixed {ms_mixed:.3f} ms, resident {ms_resident:.3f} ms per call "
          f"(published CUDA float {pub['cuda_float']} ms, mixed {pub['cuda_mixed']} ms)", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import pc_oracle
        threads = cpu_threads()
        pc_oracle.set_threads(threads)
        P = [1.0] * len(sizes)
        xs = np.stack(inputs)
        ms_batched = median_ms_of(lambda: pc_oracle.batched_relax(sizes, "tanh", eta, W, b, P, xs, T), CPU_REPS)
        pc_oracle.set_threads(1)
        ms_loop = median_ms_of(lambda: [pc_oracle.batched_relax(sizes, "tanh", eta, W, b, P, xs[i:i + 1], T)
                                        for i in range(B)], CPU_REPS)
        cpu = {"value": B * T / (ms_batched * 1e-3), "unit": "sample-steps/s", "cores": threads,
               **host_fields(threads), "kind": "port",
               "batched_ms": ms_batched, "per_sample_loop_ms": ms_loop, "per_sample_loop_threads": 1,
               "sample": f"the whole workload: oracle batched fp32 relaxation of the {B} inputs x {T} steps on "
                         f"{threads} threads (median of {CPU_REPS} after 1 warm-up), and the per-sample loop "
                         f"({B} batch-1 settlings, 1 thread)"}
        print(f"# pub cpu: batched {ms_batched:.1f} ms on {threads} threads, per-sample loop {ms_loop:.1f} ms",
              file=sys.stderr, flush=True)
    rec = {
        "metric": "relaxed samples*steps/sec at 1 GPU and % of MFMA/HBM roofline",
        "value": B * T / (ms_float * 1e-3), "unit": "sample-steps/s", "n_gpus": 1, "steps": reps, "warmup": 1,
        "ms_per_step": ms_float, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded Xavier-normal weights, N(0,1) inputs)",
        "config": {"workload": f"pub: {topology(sizes)} tanh f32, B={B}, T={T}, eta={eta}, host arrays through "
                               "BatchedPcForward.infer_get_top_batch (tools/MixedPrecisionBench/Program.cs:75-127)",
                   "batch": B, "relax_steps": T, "layer_sizes": sizes, "parallelism": "single GPU"},
        "ms_per_call": {"dropin_float": ms_float, "dropin_mixed_f16": ms_mixed, "device_resident_float": ms_resident},
        "published_ms": {**pub, "hardware": "Ryzen-class CPU + RTX 4070 SUPER",
                         "source": "PredicitiveCoding/ROADMAP-MixedPrecision.md:99"},
        "speedup_vs_published": {"cuda_float": pub["cuda_float"] / ms_float,
                                 "cuda_mixed": pub["cuda_mixed"] / ms_mixed,
                                 "cpu_batched": pub["cpu_batched"] / ms_float},
        "cpu_baseline": cpu,
    }
    if not standalone:
        for k in ("metric", "n_gpus", "higher_is_better", "scaling", "vs_baseline"):
            rec.pop(k)
    return rec


def vendor_gemm_context(sizes, B, dtype, reps=5, ramp_s=0.15):
    """The vendor library on the same box, in the same run: hipBLASLt (through
    torch.mm) computing the plain products of one error phase -- for every
    layer l, [B x s_l] @ [s_l x s_{l-1}] in `dtype`, each layer with its own
    operands and output, no epilogue.  Context for the roofline fraction of
    the fused phases (what a library GEMM of the same shapes reaches on this
    power-limited part), never a number this build reports as its own.
    Warm-up runs past the clock's ramp at process start (~50 ms) before the
    timed passes; HIP events on torch's stream, on which the products run."""
    import torch
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    L = len(sizes)
    A = [torch.randn((B, sizes[l]), device="cuda", dtype=tdt, generator=gen) for l in range(1, L)]
    Wt = [(torch.randn((sizes[l], sizes[l - 1]), device="cuda", dtype=torch.float32, generator=gen)
           * sizes[l] ** -0.5).to(tdt) for l in range(1, L)]
    out = [torch.empty((B, sizes[l - 1]), device="cuda", dtype=tdt) for l in range(1, L)]

    def one_phase():
        for a, w, o in zip(A, Wt, out):
            torch.mm(a, w, out=o)

    one_phase()   # the library's first calls choose and load their kernels
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 1
    while n < 3 or time.perf_counter() - t0 < ramp_s:
        one_phase()
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        one_phase()
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_time(e1) / reps
    flop = 2.0 * B * sum(sizes[l] * sizes[l - 1] for l in range(1, L))
    rec = {"library": f"hipBLASLt via torch.mm (torch {torch.__version__})", "ms_per_phase": ms,
           "tflops": flop / (ms * 1e-3) / 1e12, "frac": flop / (ms * 1e-3) / PEAK[dtype],
           "what": f"the plain {dtype} products of one error phase ({L - 1} layers, {dtype} out, no epilogue), "
                   f"mean of {reps} passes after {n} warm-up passes"}
    del A, Wt, out
    torch.cuda.empty_cache()
    return rec


def bench_settle(args, name, cfg, steps, warmup, cpu_budget, pcie=False):
    """One fixed-batch settling workload (c1, c2, c3, c5, c5s): `steps` timed
    passes of pcd_pc_relax on inputs resident in HBM after `warmup` untimed
    ones, the per-phase roofline from HIP events, optionally the same pass
    with host input and output (pcie), and the CPU baseline.  Returns the
    record."""
    import torch
    from predicitivecoding_amd import GenerativeSnapshot, PcDeviceModel
    sizes, B, T = cfg["sizes"], cfg["batch"], cfg["T"]
    print(f"# bench {name}: sizes={sizes} B={B} T={T} dtype={cfg['dtype']}", file=sys.stderr, flush=True)
    W, b = make_weights(cfg)
    snap = GenerativeSnapshot(sizes, cfg["act"], cfg["eta"], 0.0, False, W, b, [1.0] * len(sizes))
    model = PcDeviceModel(snap, cfg["dtype"])
    apply_options(model, args)
    if args.tile_order >= 0:
        model.set_option("tile_order", args.tile_order)
    if args.tile:
        model.set_option("tile", args.tile)
        if args.tile_n:
            model.set_option("tile_n", args.tile_n)
    x = make_inputs(cfg)
    top = torch.empty((B, sizes[-1]), device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()

    def one_pass():
        model.relax_device(x.data_ptr(), B, T, top.data_ptr())

    for _ in range(warmup):
        one_pass()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        one_pass()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / steps
    value = B * T * steps / elapsed
    print(f"# timed {steps} passes: {ms_per_step:.3f} ms/pass, {value:.4g} sample-steps/s",
          file=sys.stderr, flush=True)

    # Roofline: the same passes again with HIP events around every phase launch
    # (eager launches on the library's stream), averaged per phase.
    model.set_option("profile", 1)
    err_ms = upd_ms = 0.0
    launches = 0
    for _ in range(max(1, min(steps, 5))):
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
    bytes_err, bytes_upd = phase_bytes(sizes, B, cfg["dtype"])
    bytes_launch = bytes_upd if dom_name == "update_phase" else bytes_err
    peak = PEAK[cfg["dtype"]]
    # The roofline the arithmetic names: HBM when the launch's FLOP per
    # algorithmic byte is below the ridge (peak FLOP/s / peak HBM bytes/s).
    if flop_launch / bytes_launch < peak / HBM_PEAK:
        achieved = bytes_launch / (dom_ms * 1e-3)
        roofline = {"bound": "hbm", "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                    "frac": achieved / HBM_PEAK, "traffic": traffic_from_profiles(name, dom_name),
                    "kernel": dom_name, "kernel_ms": dom_ms, "error_phase_ms": err_ms, "update_phase_ms": upd_ms,
                    "bytes_per_launch": bytes_launch, "flop_per_launch": flop_launch,
                    "mfma_frac": flop_launch / (dom_ms * 1e-3) / peak, "launches_timed": launches}
        print(f"# roofline: error {err_ms:.4f} ms, update {upd_ms:.4f} ms per launch; {dom_name} at "
              f"{achieved / 1e9:.0f} GB/s = {100 * achieved / HBM_PEAK:.1f}% of HBM peak", file=sys.stderr,
              flush=True)
    else:
        achieved = flop_launch / (dom_ms * 1e-3)
        roofline = {"bound": "mfma", "achieved": achieved / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s",
                    "frac": achieved / peak, "traffic": traffic_from_profiles(name, dom_name),
                    "kernel": dom_name, "kernel_ms": dom_ms, "error_phase_ms": err_ms, "update_phase_ms": upd_ms,
                    "flop_per_launch": flop_launch, "bytes_per_launch": bytes_launch, "launches_timed": launches,
                    "path_frac": (flops_per_sample_step(sizes) * value) / peak,
                    # the same launch against the HBM roofline: algorithmic bytes / duration
                    "hbm_achieved_GBps": bytes_launch / (dom_ms * 1e-3) / 1e9,
                    "hbm_frac": bytes_launch / (dom_ms * 1e-3) / HBM_PEAK}
        print(f"# roofline: error {err_ms:.4f} ms, update {upd_ms:.4f} ms per launch; {dom_name} at "
              f"{achieved / 1e12:.1f} TFLOP/s = {100 * achieved / peak:.1f}% of peak, "
              f"{bytes_launch / (dom_ms * 1e-3) / 1e9:.0f} GB/s algorithmic", file=sys.stderr, flush=True)
    roofline.update(traffic_fields(sizes, B, cfg["dtype"]))
    if roofline["bound"] == "mfma" and cfg["dtype"] in ("bf16", "f16") and not (args.no_vendor or args.no_extra):
        roofline["vendor_gemm"] = vendor_gemm_context(sizes, B, cfg["dtype"])
        v = roofline["vendor_gemm"]
        print(f"# vendor GEMM (same shapes, plain): {v['ms_per_phase']:.4f} ms per phase, "
              f"{v['tflops']:.0f} TFLOP/s = {100 * v['frac']:.1f}% of peak", file=sys.stderr, flush=True)

    pcie_rec = None
    if pcie:
        # The same passes with the input on the host and the top states back
        # on the host (pinned buffers): one H2D of x0 and one D2H of the top
        # per pass, as a caller handing over host arrays pays.  Reported beside
        # `value`, which keeps the inputs resident in HBM.
        x_pin = torch.empty((B, sizes[0]), dtype=torch.float32, pin_memory=True)
        x_pin.copy_(x)
        top_pin = torch.empty((B, sizes[-1]), dtype=torch.float32, pin_memory=True)
        torch.cuda.synchronize()
        n_pcie = max(1, min(steps, 5))
        t0 = time.perf_counter()
        for _ in range(n_pcie):
            x.copy_(x_pin, non_blocking=True)
            one_pass()
            top_pin.copy_(top, non_blocking=True)
            torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / n_pcie
        pcie_rec = {"value": B * T / dt, "unit": "sample-steps/s", "ms_per_step": dt * 1e3, "passes": n_pcie,
                    "h2d_bytes": B * sizes[0] * 4, "d2h_bytes": B * sizes[-1] * 4,
                    "what": "host x0 (pinned) -> H2D -> settle -> D2H top (pinned) -> synchronize, per pass"}
        print(f"# pcie-inclusive: {dt * 1e3:.3f} ms/pass, {B * T / dt:.4g} sample-steps/s", file=sys.stderr,
              flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        x_host = x.cpu().numpy()
        cpu = cpu_baseline(cfg, W, b, x_host, cpu_budget)
        print(f"# cpu baseline: {cpu['value']:.4g} sample-steps/s on {cpu['cores']} threads", file=sys.stderr,
              flush=True)

    rec = {
        "metric": "relaxed samples*steps/sec at 1 GPU and % of MFMA/HBM roofline",
        "value": value,
        "unit": "sample-steps/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded random weights and inputs)",
        "config": {"workload": f"{name}: {topology(sizes)} {ACT_NAME[cfg['act']]} "
                               f"{cfg['dtype']}, B={B}, T={T}, eta={cfg['eta']}",
                   "batch": B, "relax_steps": T, "layer_sizes": sizes, "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if pcie_rec is not None:
        rec["pcie_inclusive"] = pcie_rec
    model.close()
    return rec




def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c5", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="leave out the c3 and published-workload records of the default (c5) line and the "
                         "same-shape hipBLASLt context (the profiling runs use it: their traces hold this library's "
                         "kernels only)")
    ap.add_argument("--no-vendor", action="store_true",
                    help="leave out the same-shape hipBLASLt context of the 16-bit settling records")
    ap.add_argument("--cpu-budget", type=float, default=20.0,
                    help="seconds the CPU baseline sample is sized for (its calibration overestimates ~2x)")
    ap.add_argument("--tile", type=int, default=0, help="force the GEMM tile rows (and columns unless --tile-n)")
    ap.add_argument("--tile-n", type=int, default=0)
    ap.add_argument("--tile-order", type=int, default=-1, help="force the tile order option (0 interleaved, 1 contiguous)")
    ap.add_argument("--option", action="append", default=[], metavar="NAME=VALUE",
                    help="set a pcd_pc_set_option relaxation option (repeatable), e.g. split_k=0")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only the copy kernel that calibrates FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--traffic-from", nargs=4, metavar=("FETCH_DIR", "WRITE_DIR", "CALIB_FETCH_DIR", "CALIB_WRITE_DIR"),
                    help="derive profiles/traffic_<config>.json from rocprofv3 --pmc output directories")
    ap.add_argument("--traffic-command", default="", help="command line recorded with --traffic-from")
    args = ap.parse_args()
    if args.traffic_from:
        traffic_from_pmc(args.config, *args.traffic_from, args.traffic_command)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build runs the relaxation on a single MI355X. The batch "
              "would shard over GPUs by rows with replicated weights and no per-step communication.",
              file=sys.stderr)
        sys.exit(2)

    if args.calibrate_copy:
        calibrate_copy()
        return

    cfg = CONFIGS[args.config]
    if args.config == "pub":
        print(json.dumps(bench_published(args, standalone=True)))
        return
    if "requests" in cfg:
        bench_ragged(args, cfg)
        return
    if "mode" in cfg:
        bench_clamped(args, cfg)
        return
    if args.config == "gemm":
        bench_gemm(args, cfg)
        return
    rec = bench_settle(args, args.config, cfg, args.steps, args.warmup, args.cpu_budget, pcie=True)
    if args.config == "c5" and not args.no_extra:
        # the configuration north_star's bf16 target is stated on, and the
        # reference's own published workload, in the same line
        rec["extra"] = {
            "c3": bench_settle(args, "c3", CONFIGS["c3"], args.steps, min(args.warmup, 3), args.cpu_budget / 2),
            "pub": bench_published(args),
        }
    print(json.dumps(rec))


if __name__ == "__main__":
    main()
