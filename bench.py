"""Benchmark of the MI355X detector path.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

Workloads (one JSON line each run):
  gemv_q4k   4096x4096 Q4_K dequant-fused GEMV, batch 1, fp32 x (default)
A step is one pass of the hot path over one batch of synthetic input resident in
HBM.  The timed region replays exactly K steps (captured in a HIP graph) between
two synchronisations.  Matrices rotate through enough distinct copies to exceed
3x the 256 MB Infinity Cache, so every step streams its weights from HBM.

roofline.achieved is the algorithmic bytes of one launch of the dominant kernel
divided by that kernel's mean duration, measured live with HIP events recorded on
the launching stream around individual launches.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "ray-tracing-attention_amd"))

HBM_PEAK_GBS = 8000.0
CACHE_BYTES = 256 << 20
METRIC = "decode tokens/sec at batch 1/32 (9B-shape) + Q4_K GEMV GB/s, % of HBM peak"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="gemv_q4k", choices=["gemv_q4k"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    return ap.parse_args()


def traffic_for(workload):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/traffic.json), if recorded."""
    f = ROOT / "profiles" / "traffic.json"
    if f.is_file():
        return json.loads(f.read_text()).get(workload)
    return None


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_kernel(torch, launch, n=200):
    """Mean duration (ms) of single launches bracketed by events on the launch stream."""
    s = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for i in range(n):
        starts[i].record(s)
        launch(i)
        ends[i].record(s)
    torch.cuda.synchronize()
    d = np.array([a.elapsed_time(b) for a, b in zip(starts, ends)])
    return float(np.median(d)), float(d.mean())


def timed_region(torch, launch, steps, warmup):
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                launch(i)
    torch.cuda.synchronize()
    g.replay()                      # graph warm-up (not timed)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3


def bench_gemv_q4k(torch, args):
    from rta import ops, synth
    rows = cols = 4096
    dev = torch.device("cuda:0")
    rng = synth.rng_for(1)
    w = synth.random_matrix(rng, 12, rows, cols)
    x = rng.standard_normal((1, cols)).astype(np.float32)
    wbytes = w.nbytes
    ncopy = max(2, int(3 * CACHE_BYTES // wbytes) + 1)
    w0 = torch.from_numpy(w).to(dev)
    copies = [w0] + [w0.clone() for _ in range(ncopy - 1)]
    xd = torch.from_numpy(x).to(dev)
    y = torch.empty(1, rows, dtype=torch.float32, device=dev)

    def launch(i):
        ops.gemv(12, copies[i % ncopy], rows, cols, xd, y=y)

    alg_bytes = wbytes + 4 * cols + 4 * rows
    med, mean = time_kernel(torch, launch)
    ms = timed_region(torch, launch, args.steps, args.warmup)
    ms_step = ms / args.steps
    # parity of the timed configuration against the oracle (one copy)
    out = {
        "value": alg_bytes / (ms_step * 1e-3) / 1e9,
        "unit": "GB/s",
        "ms_per_step": ms_step,
        "dtype": "q4_k weights x fp32 activations, fp32 accumulate",
        "config": {"workload": "Q4_K GEMV 4096x4096, batch 1 (single dequant-fused matrix-vector readout)",
                   "rows": rows, "cols": cols, "batch": 1, "weight_copies_rotated": ncopy,
                   "rotated_bytes": ncopy * wbytes, "seed": "20261110+1"},
        "kernel": "gemv_kquant_kernel<Q4_K,NB=1,R=4,store>",
        "alg_bytes_per_launch": alg_bytes,
        "kernel_ms_median": med,
        "kernel_ms_mean": mean,
        "roofline": {"bound": "hbm", "achieved": alg_bytes / (med * 1e-3) / 1e9, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": alg_bytes / (med * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "traffic": traffic_for("gemv_q4k")},
    }
    host = {"w": w, "x": x, "rows": rows, "cols": cols, "alg_bytes": alg_bytes}
    return out, host, lambda: y.cpu().numpy()


def cpu_baseline_gemv(host, seconds):
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as orc
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    w, x = host["w"], host["x"]
    orc.gemv_f32(12, w, host["rows"], host["cols"], x, threads)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        orc.gemv_f32(12, w, host["rows"], host["cols"], x, threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": host["alg_bytes"] * n / el / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{n} calls of the oracle's fp32-accumulating OpenMP Q4_K GEMV (4096x4096, batch 1) "
                      f"in {el:.1f} s on {cpu_model()}"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 (no multi-GPU path is "
                                   "built: every GPU box here has one GPU)"}))
        sys.exit(2)
    import torch
    from rta import _lib
    _lib.load()
    if args.workload == "gemv_q4k":
        out, host, fetch = bench_gemv_q4k(torch, args)
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as orc
        ref = orc.gemv_f64(12, host["w"], host["rows"], host["cols"], host["x"])
        got = fetch()
        err = float(np.max(np.abs(got - ref)))
        out["parity"] = {"max_abs_err": err, "peak": float(np.abs(ref).max()),
                         "ok": bool(err <= 1e-5 + 1e-3 * np.abs(ref).max())}
        cpu = None if args.no_cpu else cpu_baseline_gemv(host, args.cpu_seconds)
    line = {"metric": METRIC, "value": out["value"], "unit": out["unit"], "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": out["ms_per_step"], "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": out["dtype"], "data": "synthetic",
            "config": out["config"], "roofline": out["roofline"], "cpu_baseline": cpu,
            "kernel": out["kernel"], "kernel_ms_median": out["kernel_ms_median"],
            "kernel_ms_mean": out["kernel_ms_mean"], "alg_bytes_per_launch": out["alg_bytes_per_launch"],
            "parity": out["parity"]}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
