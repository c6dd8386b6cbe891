"""Benchmark of the MI355X detector path.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--batch B] [--no-cpu]

Workloads (one JSON line per run):
  gemv_q4k    4096x4096 Q4_K dequant-fused GEMV, batch 1, fp32 x
  mlp         SwiGLU MLP 2048 -> 6144 -> 2048, gate/up Q4_K, down Q6_K, --batch rows
  lm_head     151936 x 2048 Q6_K vocabulary readout + margin argmax, --batch rows
  attention   GQA decode attention, 16 sequences, contexts log-uniform in [512, 32768],
              16 q / 4 kv heads, hd 128, K Q6_K / V Q4_K history, RoPE theta 1e6 on q
  proj        one projection --rows x --cols in --fmt q4k|q6k for --batch rows
  decode      9B-shape hybrid decode step (24 delta-net + 8 attention layers), --batch sequences
              (default 32), tokens/s                                          (default)
  copy_calib  plain device-to-device copy of known size (PMC byte-counter calibration)

A step is one pass of the hot path over one batch of synthetic input resident in
HBM.  The timed region replays exactly K steps (captured in a HIP graph) between
two synchronisations.  Weights (and the attention history) rotate through enough
distinct copies to exceed 3x the 256 MB Infinity Cache, so every step streams
them from HBM.

roofline.achieved = algorithmic bytes of one launch of the dominant kernel / that
kernel's mean duration, measured with HIP events recorded on the launching
stream around a graph of back-to-back launches of that kernel.  For the decode
step the dominant kernel is the one with the largest share of a step (calls per
step x mean duration); every timed kernel is listed under "kernels".
read_ceiling: the achievable HBM read rate (a streaming-read kernel over 1 GiB);
roofline.frac_of_ceiling = achieved / that rate, beside frac = achieved / 8 TB/s.
read_ceiling_at_size (gemv_q4k): the same kernel reading the GEMV's byte count once per
launch, timed like the GEMV; roofline.frac_of_size_ceiling = achieved / its rate.
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
Q4_K, Q6_K = 12, 14


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 64 for decode, else 1000)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (default 4 for decode, else 100)")
    ap.add_argument("--workload", default="decode",
                    choices=["gemv_q4k", "mlp", "lm_head", "attention", "proj", "decode", "copy_calib"])
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--rows", type=int, default=12288, help="proj workload: output rows")
    ap.add_argument("--cols", type=int, default=4096, help="proj workload: input columns")
    ap.add_argument("--fmt", default="q4k", choices=["q4k", "q6k"], help="proj workload: weight format")
    ap.add_argument("--packed", action="store_true",
                    help="proj / mlp / lm_head / decode: weights packed once by rta_pack (tiled layout, matrix cores)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a graph replay")
    ap.add_argument("--no-companions", action="store_true",
                    help="decode: skip the batch-1 step and the Q4_K GEMV figures reported beside it")
    return ap.parse_args()


def traffic_for(key):
    """HBM bytes per launch of a kernel (key: the workload, or the workload and the kernel's
    short name, "decode/gate/up"), from rocprofv3 --pmc runs (profiles/traffic.json)."""
    f = ROOT / "profiles" / "traffic.json"
    if f.is_file():
        return json.loads(f.read_text()).get(key)
    return None


def read_ceiling(torch, n_bytes=1 << 30):
    """Achievable HBM read rate: the streaming-read kernels of lib/librta_ceiling.so over one
    1 GiB buffer (4x the 256 MB last-level cache), 20 back-to-back launches between HIP
    events on one stream, for each variant and a few grid sizes; the best rate is the
    ceiling."""
    import ctypes
    path = ROOT / "ray-tracing-attention_amd" / "lib" / "librta_ceiling.so"
    if not path.is_file():
        return None
    lib = ctypes.CDLL(str(path))
    lib.rta_ceiling_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_void_p]
    lib.rta_ceiling_stream_read.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    buf = torch.empty(n_bytes, dtype=torch.uint8, device=dev).fill_(7)
    out = torch.empty(65536, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream()
    names = ["4 loads per trip", "8 loads per trip", "4 non-temporal loads", "8 non-temporal loads"]
    best = (0.0, 0, 0)
    for variant in range(4):
        for blocks in (2048, 8192, 32768):
            def launch():
                rc = lib.rta_ceiling_stream_read(buf.data_ptr(), n_bytes, out.data_ptr(), blocks, variant,
                                                 s.cuda_stream)
                if rc:
                    raise RuntimeError(f"rta_ceiling_stream_read failed: {rc}")
            for _ in range(3):
                launch()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(s)
            for _ in range(20):
                launch()
            b.record(s)
            torch.cuda.synchronize()
            best = max(best, (n_bytes / (a.elapsed_time(b) / 20 * 1e-3) / 1e9, blocks, variant))
    del buf
    return {"kernel": f"stream_read_kernel, {names[best[2]]} (lib/librta_ceiling.so)", "bytes": n_bytes,
            "gbs": best[0], "frac_of_peak": best[0] / HBM_PEAK_GBS, "blocks": best[1]}


def read_ceiling_at(torch, n_bytes):
    """What one launch that reads n_bytes once costs on this GPU: the streaming-read kernels of
    lib/librta_ceiling.so over rotated n_bytes buffers (more than 3x the last-level cache in
    all, one buffer per launch), 200 launches in a HIP graph timed as time_kernel times the
    readouts; the best mean launch duration over the variants and grid sizes."""
    import ctypes
    path = ROOT / "ray-tracing-attention_amd" / "lib" / "librta_ceiling.so"
    if not path.is_file():
        return None
    lib = ctypes.CDLL(str(path))
    lib.rta_ceiling_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_void_p]
    lib.rta_ceiling_stream_read.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    n = (n_bytes + 15) // 16 * 16
    copies = [torch.empty(n, dtype=torch.uint8, device=dev).fill_(7)
              for _ in range(int(min(256, max(2, 3 * CACHE_BYTES // n + 1))))]
    out = torch.empty(65536, dtype=torch.int32, device=dev)
    best = None
    for variant in range(4):
        for blocks in (256, 512, 1024, 2048, 4096):
            def launch(i):
                rc = lib.rta_ceiling_stream_read(copies[i % len(copies)].data_ptr(), n, out.data_ptr(), blocks,
                                                 variant, torch.cuda.current_stream().cuda_stream)
                if rc:
                    raise RuntimeError(f"rta_ceiling_stream_read failed: {rc}")
            ms = time_kernel(torch, launch)
            if best is None or ms < best[0]:
                best = (ms, blocks, variant)
    del copies
    return {"bytes": n, "us": best[0] * 1e3, "gbs": n / (best[0] * 1e-3) / 1e9, "blocks": best[1],
            "variant": best[2]}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def omp_threads():
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def rotation(torch, host_array, dev, min_total=3 * CACHE_BYTES, max_copies=256):
    """Distinct device copies of host_array totalling more than min_total bytes."""
    t0 = torch.from_numpy(np.ascontiguousarray(host_array)).to(dev)
    n = int(min(max_copies, max(2, min_total // t0.numel() + 1)))
    return [t0] + [t0.clone() for _ in range(n - 1)]


def time_kernel(torch, launch, n=200):
    """Mean duration (ms) of one launch of the dominant kernel: n back-to-back launches captured
    in a HIP graph, replayed between two events recorded on the launching stream."""
    for i in range(10):
        launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(n):
                launch(i)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(s)
        g.replay()
        b.record(s)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / n


def timed_region(torch, step, steps, warmup, eager=False):
    """Exactly `steps` steps captured in one graph; returns wall ms of one replay."""
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    if eager:
        t0 = time.perf_counter()
        for i in range(steps):
            step(i)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                step(i)
    torch.cuda.synchronize()
    g.replay()                      # graph warm-up (not timed)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3


def timed_replays(torch, step, steps, warmup):
    """One step captured in a graph and replayed `steps` times; returns wall ms of all replays."""
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            step(0)
    torch.cuda.synchronize()
    g.replay()                      # graph warm-up (not timed)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3


def cpu_time(fn, seconds):
    fn()  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return n, el


def close(got, ref):
    """The float bar, max|got - ref| <= 1e-5 + 1e-3 max|ref| per tensor, and beside it the
    fraction of elements passing the elementwise allclose(rtol=1e-3, atol=1e-5) test."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    err = float(np.max(np.abs(got - ref)))
    peak = float(np.max(np.abs(ref)))
    elem = float(np.mean(np.abs(got - ref) <= 1e-5 + 1e-3 * np.abs(ref)))
    return {"max_abs_err": err, "peak": peak, "ok": bool(err <= 1e-5 + 1e-3 * peak),
            "allclose_1e-3_1e-5_pass_fraction": elem}


# ------------------------------------------------------------------ workloads ----
def w_gemv_q4k(torch, args, orc):
    from rta import ops, synth
    rows = cols = 4096
    dev = torch.device("cuda:0")
    rng = synth.rng_for(1)
    w = synth.random_matrix(rng, Q4_K, rows, cols)
    x = rng.standard_normal((1, cols)).astype(np.float32)
    copies = rotation(torch, w, dev)
    xd = torch.from_numpy(x).to(dev)
    y = torch.empty(1, rows, dtype=torch.float32, device=dev)

    def step(i):
        ops.gemv(Q4_K, copies[i % len(copies)], rows, cols, xd, y=y)

    alg = w.nbytes + 4 * cols + 4 * rows
    res = {"alg_bytes": alg, "kernel": "gemv_b1_kernel<Q4_K,R=2,store,KW=1>", "step": step, "kernel_launch": step,
           "unit": "GB/s", "value_from_ms": lambda ms: alg / (ms * 1e-3) / 1e9,
           "dtype": "q4_k weights x fp32 activations, fp32 accumulate",
           "config": {"workload": "Q4_K GEMV 4096x4096, batch 1 (single dequant-fused matrix-vector readout)",
                      "rows": rows, "cols": cols, "batch": 1, "weight_copies_rotated": len(copies),
                      "seed": "20261110+1"}}

    def check():
        step(0)
        return close(y.cpu().numpy(), orc.gemv_f64(Q4_K, w, rows, cols, x))

    def cpu(seconds):
        t = omp_threads()
        n, el = cpu_time(lambda: orc.gemv_f32(Q4_K, w, rows, cols, x, t), seconds)
        return {"value": alg * n / el / 1e9, "unit": "GB/s", "cores": t, "kind": "port",
                "sample": f"{n} calls of the oracle's fp32-accumulating OpenMP Q4_K GEMV 4096x4096 batch 1 "
                          f"in {el:.1f} s on {cpu_model()}"}
    res["check"], res["cpu"] = check, cpu
    return res


def w_mlp(torch, args, orc):
    from rta import ops, synth
    hidden, inter = 2048, 6144
    batch = args.batch or 1
    dev = torch.device("cuda:0")
    rng = synth.rng_for(2)
    wg = synth.random_matrix(rng, Q4_K, inter, hidden)
    wu = synth.random_matrix(rng, Q4_K, inter, hidden)
    wd = synth.random_matrix(rng, Q6_K, hidden, inter)
    x = rng.standard_normal((batch, hidden)).astype(np.float32)
    packed = np.concatenate([wg.ravel(), wu.ravel(), wd.ravel()])
    copies = rotation(torch, packed, dev)
    ng, nd = wg.size, wd.size
    fm = (Q4_K, Q4_K, Q6_K)
    mats = [(c[:ng], c[ng:2 * ng], c[2 * ng:]) for c in copies]
    kfm = fm
    if args.packed:
        mats = [(ops.pack(Q4_K, g_, inter, hidden), ops.pack(Q4_K, u_, inter, hidden), ops.pack(Q6_K, d_, hidden, inter))
                for g_, u_, d_ in mats]
        kfm = tuple(f | ops.TILED for f in fm)
        del copies
    xd = torch.from_numpy(x).to(dev)
    act = torch.empty(batch, inter, dtype=torch.float32, device=dev)
    y = torch.empty(batch, hidden, dtype=torch.float32, device=dev)
    ws = torch.empty(max(1, ops.mlp_workspace_bytes(kfm[0], kfm[2], hidden, inter, batch)), dtype=torch.uint8,
                     device=dev)

    def step(i):
        g_, u_, d_ = mats[i % len(mats)]
        ops.mlp_swiglu(kfm, g_, u_, d_, hidden, inter, xd, y=y, act=act, workspace=ws)

    alg = packed.nbytes + batch * (hidden * 4 + inter * 4 + hidden * 4)
    res = {"alg_bytes": alg, "kernel": "gate/up SwiGLU pair: " + readout_name("Q4_K", inter, hidden, batch, args.packed, True)
           + "; down: " + readout_name("Q6_K", hidden, inter, batch, args.packed), "step": step,
           "kernel_launch": step, "unit": "GB/s", "value_from_ms": lambda ms: alg / (ms * 1e-3) / 1e9,
           "dtype": "q4_k/q6_k weights x fp32 activations, fp32 accumulate",
           "config": {"workload": f"SwiGLU MLP 2048->6144->2048 (gate/up Q4_K, down Q6_K), batch {batch}"
                                  + (" (packed tiles)" if args.packed else ""),
                      "hidden": hidden, "intermediate": inter, "batch": batch, "weight_copies_rotated": len(mats),
                      "seed": "20261110+2"}}

    def check():
        step(0)
        ract, ry = orc.mlp_swiglu(fm, wg, wu, wd, hidden, inter, x)
        a, b = close(act.cpu().numpy(), ract), close(y.cpu().numpy(), ry)
        return {"activation": a, "output": b, "ok": a["ok"] and b["ok"]}

    def cpu(seconds):
        n, el = cpu_time(lambda: orc.mlp_swiglu(fm, wg, wu, wd, hidden, inter, x), seconds)
        return {"value": alg * n / el / 1e9, "unit": "GB/s", "cores": omp_threads(), "kind": "port",
                "sample": f"{n} calls of the oracle's fp64 SwiGLU MLP (batch {batch}) in {el:.1f} s on {cpu_model()}"}
    res["check"], res["cpu"] = check, cpu
    return res


def readout_name(fmt_name, rows, cols, batch, packed, pair=False):
    """The kernel a projection readout runs (the library's dispatch, for the bench line's
    label): packed tiles on the matrix cores; GGUF rows on the batch-1 readout, the
    vector-ALU batch readout, or the matrix cores from batch 5 (3 at 2^25+ weights, 2 at
    2^27+ weights, a SwiGLU pair counting both matrices)."""
    if packed:
        return f"gemm_tiled_kernel<{fmt_name}> (packed tiles, matrix cores)"
    if batch == 1:
        return f"gemv_b1_kernel<{fmt_name}> (GGUF rows, vector ALUs)"
    weights = rows * cols * (2 if pair else 1)
    if batch >= 5 or (batch >= 3 and weights >= 1 << 25) or (batch >= 2 and weights >= 1 << 27):
        return f"xprep_kernel + gemm_mfma_kernel<{fmt_name}> (GGUF rows, matrix cores)"
    return f"gemv_kquant_kernel<{fmt_name}> (GGUF rows, vector ALUs)"


def w_lm_head(torch, args, orc):
    from rta import ops, synth
    vocab, hidden = 151936, 2048
    batch = args.batch or 1
    dev = torch.device("cuda:0")
    rng = synth.rng_for(4)
    w = synth.random_matrix(rng, Q6_K, vocab, hidden)
    h = (rng.standard_normal((batch, hidden)) * 2.0).astype(np.float32)
    copies = rotation(torch, w, dev)
    kfmt = Q6_K
    if args.packed:
        copies = [ops.pack(Q6_K, c, vocab, hidden) for c in copies]
        kfmt = Q6_K | ops.TILED
    hd = torch.from_numpy(h).to(dev)
    logits = torch.empty(batch, vocab, dtype=torch.float32, device=dev)
    ids = torch.empty(batch, dtype=torch.int32, device=dev)
    ws = torch.empty(ops.lm_head_workspace_bytes(kfmt, vocab, hidden, batch), dtype=torch.uint8, device=dev)
    gws = torch.empty(max(1, ops.gemv_workspace_bytes(kfmt, vocab, hidden, batch)), dtype=torch.uint8, device=dev)

    def step(i):
        ops.lm_head(kfmt, copies[i % len(copies)], vocab, hidden, hd, margin=1e-4, workspace=ws, logits=logits,
                    ids=ids)

    def readout(i):  # the dominant kernel alone: the Q6_K logits GEMV
        ops.gemv(kfmt, copies[i % len(copies)], vocab, hidden, hd, y=logits, workspace=gws)

    alg = w.nbytes + batch * (hidden * 4 + vocab * 4 + 4)
    alg_k = w.nbytes + batch * (hidden * 4 + vocab * 4)
    res = {"alg_bytes": alg, "alg_bytes_kernel": alg_k,
           "kernel": "Q6_K logits readout: " + readout_name("Q6_K", vocab, hidden, batch, args.packed),
           "step": step, "kernel_launch": readout, "unit": "GB/s", "value_from_ms": lambda ms: alg / (ms * 1e-3) / 1e9,
           "dtype": "q6_k weights x fp32 activations, fp32 accumulate",
           "config": {"workload": f"LM head 151936x2048 Q6_K + margin argmax, batch {batch}"
                                  + (" (packed tiles)" if args.packed else ""), "vocab": vocab,
                      "hidden": hidden, "batch": batch, "weight_copies_rotated": len(copies),
                      "seed": "20261110+4"}}

    def check():
        step(0)
        lg = logits.cpu().numpy()
        ref = orc.gemv_f64(Q6_K, w, vocab, hidden, h)
        c = close(lg, ref)
        got_ids = ids.cpu().numpy().view(np.uint32)
        rule = [orc.argmax_margin_f32(lg[b], 1e-4) for b in range(batch)]
        c["ids_match_rule"] = bool(list(got_ids) == rule)
        c["ids_match_oracle"] = bool(list(got_ids) == [orc.argmax_margin_f64(ref[b], 1e-4) for b in range(batch)])
        c["ok"] = c["ok"] and c["ids_match_rule"]
        return c

    def cpu(seconds):
        t = omp_threads()
        n, el = cpu_time(lambda: orc.gemv_f32(Q6_K, w, vocab, hidden, h, t), seconds)
        return {"value": alg * n / el / 1e9, "unit": "GB/s", "cores": t, "kind": "port",
                "sample": f"{n} calls of the oracle's fp32 OpenMP Q6_K readout 151936x2048 batch {batch} "
                          f"in {el:.1f} s on {cpu_model()}"}
    res["check"], res["cpu"] = check, cpu
    return res


def w_attention(torch, args, orc):
    from rta import ops, synth
    nseq, hq, hkv, hd = 16, 16, 4, 128
    dev = torch.device("cuda:0")
    rng = synth.rng_for(3)
    ctx = synth.log_uniform_lengths(rng, nseq, 512, 32768)
    base = np.concatenate([[0], np.cumsum(ctx)[:-1]]).astype(np.int64)
    total = int(ctx.sum())
    kvw = hkv * hd
    packets = synth.random_packets(rng, total, kvw, Q6_K, Q4_K)
    q = rng.standard_normal((nseq, hq, hd)).astype(np.float32)
    copies = rotation(torch, packets, dev)
    qd = torch.from_numpy(q).to(dev)
    qr = torch.empty_like(qd)
    pos = torch.from_numpy(ctx - 1).to(dev)
    based = torch.from_numpy(base).to(dev)
    ctxd = torch.from_numpy(ctx.astype(np.int32)).to(dev)
    cap = int(ctx.max())
    ws = torch.empty(ops.decode_attention_workspace_bytes(nseq, hq, hkv, hd, cap), dtype=torch.uint8, device=dev)
    out = torch.empty_like(qd)

    def attn(i):
        ops.decode_attention(qr, copies[i % len(copies)], Q6_K, Q4_K, based, ctxd, cap, cap, hkv, workspace=ws,
                             out=out)

    def step(i):
        qr.copy_(qd)
        ops.rope(qr, pos, theta=1e6)
        attn(i)

    alg = total * (2 * 354) + 2 * nseq * hq * hd * 4
    res = {"alg_bytes": alg, "kernel": "attn_chunk_mma6_kernel<G=4> (Q6_K keys, Q4_K values, matrix cores) + attn_merge_kernel", "step": step,
           "kernel_launch": attn, "unit": "GB/s", "value_from_ms": lambda ms: alg / (ms * 1e-3) / 1e9,
           "dtype": "q6_k keys / q4_k values x fp32 queries, fp32 softmax",
           "config": {"workload": "GQA decode attention, 16 seq, ctx log-uniform [512,32768], 16q/4kv heads, "
                                  "hd 128, K Q6_K V Q4_K, RoPE 1e6",
                      "contexts": [int(c) for c in ctx], "sum_context": total, "history_copies_rotated": len(copies),
                      "seed": "20261110+3"}}

    def check():
        step(0)
        qrot = np.stack([orc.rope(q[s], ctx[s] - 1, theta=1e6) for s in range(nseq)])
        # sampled: the oracle over all 16 sequences at full length takes minutes; check 4 of them
        pick = [int(i) for i in np.argsort(ctx)[[0, 5, 10, 15]]]
        sub_base = np.concatenate([[0], np.cumsum(ctx[pick])[:-1]]).astype(np.int64)
        sub_pk = np.concatenate([packets[base[s]:base[s] + ctx[s]] for s in pick])
        ro, rm, rz = orc.decode_attention(qrot[pick], sub_pk, Q6_K, Q4_K, sub_base, ctx[pick], cap, hkv)
        c = close(out.cpu().numpy()[pick], ro)
        c["sequences_checked"] = pick
        return c

    def cpu(seconds):
        sub = int(np.argmin(ctx))
        qrot = orc.rope(q[sub], ctx[sub] - 1, theta=1e6)[None]
        pk = packets[base[sub]:base[sub] + ctx[sub]]
        n, el = cpu_time(lambda: orc.decode_attention(qrot, pk, Q6_K, Q4_K, [0], [ctx[sub]], cap, hkv), seconds)
        by = int(ctx[sub]) * 708 + 2 * hq * hd * 4
        return {"value": by * n / el / 1e9, "unit": "GB/s", "cores": omp_threads(), "kind": "port",
                "sample": f"{n} oracle attention calls over one sequence of {int(ctx[sub])} positions "
                          f"(16 heads) in {el:.1f} s on {cpu_model()}"}
    res["check"], res["cpu"] = check, cpu
    return res


def w_proj(torch, args, orc):
    """One dequant-fused projection y = W x of --rows x --cols in --fmt (q4k / q6k) for --batch rows."""
    from rta import ops, synth
    fmt = {"q4k": Q4_K, "q6k": Q6_K}[args.fmt]
    rows, cols, batch = args.rows, args.cols, args.batch or 1
    dev = torch.device("cuda:0")
    rng = synth.rng_for(5)
    w = synth.random_matrix(rng, fmt, rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    copies = rotation(torch, w, dev)
    kfmt = fmt
    if args.packed:
        copies = [ops.pack(fmt, c, rows, cols) for c in copies]
        kfmt = fmt | ops.TILED
    xd = torch.from_numpy(x).to(dev)
    y = torch.empty(batch, rows, dtype=torch.float32, device=dev)
    ws = torch.empty(max(1, ops.gemv_workspace_bytes(kfmt, rows, cols, batch)), dtype=torch.uint8, device=dev)

    def step(i):
        ops.gemv(kfmt, copies[i % len(copies)], rows, cols, xd, y=y, workspace=ws)

    alg = w.nbytes + batch * 4 * (cols + rows)
    res = {"alg_bytes": alg, "kernel": "dequant-fused projection (matrix cores from batch 5; 3 at 2^25+ weights, 2 at 2^27+)", "step": step,
           "kernel_launch": step, "unit": "GB/s", "value_from_ms": lambda ms: alg / (ms * 1e-3) / 1e9,
           "dtype": f"{args.fmt} weights x fp32 activations, fp32 accumulate",
           "config": {"workload": f"{args.fmt.upper()} projection {rows}x{cols}, batch {batch}"
                                  + (" (packed tiles)" if args.packed else ""), "rows": rows,
                      "cols": cols, "batch": batch, "weight_copies_rotated": len(copies), "seed": "20261110+5"}}

    def check():
        step(0)
        sub = min(rows, 4096)   # the fp64 oracle over the first rows
        return close(y.cpu().numpy()[:, :sub], orc.gemv_f64(fmt, w[:sub], sub, cols, x))

    def cpu(seconds):
        t = omp_threads()
        sub = min(rows, 4096)
        n, el = cpu_time(lambda: orc.gemv_f32(fmt, w[:sub], sub, cols, x, t), seconds)
        by = w[:sub].nbytes + batch * 4 * (cols + sub)
        return {"value": by * n / el / 1e9, "unit": "GB/s", "cores": t, "kind": "port",
                "sample": f"{n} calls of the oracle's fp32 OpenMP projection over {sub} rows x {cols}, batch {batch}"
                          f" in {el:.1f} s on {cpu_model()}"}
    res["check"], res["cpu"] = check, cpu
    return res


def step_kernels(torch, shape, batch, dev, packed):
    """The decode step's readouts and its attention as separate calls of the C ABI, at the
    step's shapes (packed readouts as the step runs them: from the x image, K slabs left), each over enough distinct (rotated) weight copies that every call
    streams its weights from HBM, on the weight layout the step runs (packed tiles read by
    the matrix-core readout, or GGUF rows read by the vector-ALU one).  Returns [(name,
    calls per step, alg bytes, launch)]."""
    from rta import model, ops
    gen = torch.Generator(device=dev)
    gen.manual_seed(20261116)
    D, FF, hq, hkv, hd = shape.hidden, shape.ff, shape.q_heads, shape.kv_heads, shape.head_dim
    S = shape.rec_heads * hd
    nfull = shape.layers // shape.full_every
    nrec = shape.layers - nfull
    P4 = Q4_K | ops.TILED if packed else Q4_K
    kern = "gemm_tiled_kernel" if packed else "gemv_b1_kernel"
    lay = "packed" if packed else "GGUF rows"
    qb = lambda fmt, rows, cols: rows * cols // 256 * (144 if fmt == Q4_K else 210)  # noqa: E731

    def copies(fmt, rows, cols, per=1):
        n = max(2, 3 * CACHE_BYTES // (per * qb(fmt, rows, cols)) + 1)
        make = lambda: model.random_kquant(fmt, rows, cols, gen, dev)  # noqa: E731
        return [[ops.pack(fmt, make(), rows, cols) if packed else make() for _ in range(per)] for _ in range(n)]

    x_d = torch.randn(batch, D, device=dev, generator=gen)
    x_ff = torch.randn(batch, FF, device=dev, generator=gen) * 0.1
    act = torch.empty(batch, FF, device=dev)
    y_d = torch.zeros(batch, D, device=dev)
    y_in = torch.empty(batch, 4 * S + 2 * shape.rec_heads, device=dev)
    y_full = torch.empty(batch, (hq + 2 * hkv) * hd, device=dev)
    ws = torch.empty(max(1, ops.mlp_workspace_bytes(P4, P4, D, FF, batch),
                         ops.gemv_workspace_bytes(P4, 4 * S + 2 * shape.rec_heads, D, batch)),
                     dtype=torch.uint8, device=dev)
    gu = copies(Q4_K, FF, D, per=2)
    dn = copies(Q4_K, D, FF)
    op = copies(Q4_K, D, hq * hd)
    rin = copies(Q4_K, 4 * S + 2 * shape.rec_heads, D)
    fin = copies(Q4_K, (hq + 2 * hkv) * hd, D)
    out = []
    if packed:
        # the step's own readout kernel: gemm_packed_kernel over the x image (built once,
        # outside the timed launches), K slabs left for the next kernel of the step
        img_d, _ = ops.image_from_rows(P4, x_d)
        ws_img = torch.empty(max(ops.image_readout_workspace_bytes(FF, D, True),
                                 ops.image_readout_workspace_bytes(4 * S + 2 * shape.rec_heads, D, False),
                                 ops.image_readout_workspace_bytes((hq + 2 * hkv) * hd, D, False)),
                             dtype=torch.uint8, device=dev)
        out.append(("gate/up: gemm_packed_kernel<Q4_K,SwiGLU> from the x image, K slabs left (rta_image_readout, "
                    "packed 2 x 12288x4096)", shape.layers, 2 * qb(Q4_K, FF, D) + 4 * batch * (D + FF),
                    lambda i: ops.image_readout(P4, ops.IMAGE_SWIGLU, gu[i % len(gu)][0], gu[i % len(gu)][1], FF, D,
                                                img_d, batch, act, reduce=False, workspace=ws_img)))
    else:
        out.append((f"gate/up: {kern}<Q4_K,SwiGLU> (rta_swiglu, {lay} 2 x 12288x4096)", shape.layers,
                    2 * qb(Q4_K, FF, D) + 4 * batch * (D + FF),
                    lambda i: ops.swiglu(P4, gu[i % len(gu)][0], gu[i % len(gu)][1], D, FF, x_d, act=act,
                                         workspace=ws)))
    ns_gu = 0
    if packed:   # the down projection's x image as the step builds it: SwiGLU of the gate/up slabs
        ws_gu = torch.empty(ops.image_readout_workspace_bytes(FF, D, True), dtype=torch.uint8, device=dev)
        ns_gu = ops.image_readout(P4, ops.IMAGE_SWIGLU, gu[0][0], gu[0][1], FF, D, img_d, batch, act,
                                  reduce=False, workspace=ws_gu)
    if ns_gu > 1:
        img_ff = ops.image_from_swiglu(P4, ws_gu.view(torch.float32), ns_gu, FF, batch)
        ws_dn = torch.empty(ops.image_readout_workspace_bytes(D, FF, False), dtype=torch.uint8, device=dev)
        out.append(("down: gemm_packed_kernel<Q4_K,accumulate> from the SwiGLU image, K slabs left "
                    "(rta_image_readout, packed 4096x12288)", shape.layers, qb(Q4_K, D, FF) + 4 * batch * (FF + 2 * D),
                    lambda i: ops.image_readout(P4, 1, dn[i % len(dn)][0], None, D, FF, img_ff, batch, y_d,
                                                reduce=False, workspace=ws_dn)))
    else:
        out.append((f"down: {kern}<Q4_K,accumulate> + slab reduce (rta_gemv, {lay} 4096x12288)", shape.layers,
                    qb(Q4_K, D, FF) + 4 * batch * (FF + 2 * D),
                    lambda i: ops.gemv(P4, dn[i % len(dn)][0], D, FF, x_ff, y=y_d, accumulate=True, workspace=ws)))
    out.append((f"O projection: {kern}<Q4_K,accumulate> + slab reduce (rta_gemv, {lay} 4096x4096)",
                shape.layers, qb(Q4_K, D, hq * hd) + 4 * batch * (hq * hd + 2 * D),
                lambda i: ops.gemv(P4, op[i % len(op)][0], D, hq * hd, x_d, y=y_d, accumulate=True, workspace=ws)))
    rw, fw = 4 * S + 2 * shape.rec_heads, (hq + 2 * hkv) * hd
    if packed:
        out.append(("recurrent in-projection: gemm_packed_kernel<Q4_K,store> from the x image, K slabs left "
                    "(rta_image_readout, packed 16448x4096)", nrec, qb(Q4_K, rw, D) + 4 * batch * (D + rw),
                    lambda i: ops.image_readout(P4, 0, rin[i % len(rin)][0], None, rw, D, img_d, batch, y_in,
                                                reduce=False, workspace=ws_img)))
        out.append(("full in-projection: gemm_packed_kernel<Q4_K,store> from the x image, K slabs left "
                    "(rta_image_readout, packed 6144x4096)", nfull, qb(Q4_K, fw, D) + 4 * batch * (D + fw),
                    lambda i: ops.image_readout(P4, 0, fin[i % len(fin)][0], None, fw, D, img_d, batch, y_full,
                                                reduce=False, workspace=ws_img)))
    else:
        out.append((f"recurrent in-projection: {kern}<Q4_K,store> (rta_gemv, {lay} 16448x4096)", nrec,
                    qb(Q4_K, rw, D) + 4 * batch * (D + rw),
                    lambda i: ops.gemv(P4, rin[i % len(rin)][0], rw, D, x_d, y=y_in, workspace=ws)))
        out.append((f"full in-projection: {kern}<Q4_K,store> (rta_gemv, {lay} 6144x4096)", nfull,
                    qb(Q4_K, fw, D) + 4 * batch * (D + fw),
                    lambda i: ops.gemv(P4, fin[i % len(fin)][0], fw, D, x_d, y=y_full, workspace=ws)))
    return out


def w_decode(torch, args, orc):
    """The 9B-shape hybrid decode step: 32 layers (3 gated delta-net : 1 full attention),
    hidden 4096, 32/8 heads x 128, 32 delta-net heads, FF 12288, Q4_K projections, Q6_K LM
    head 151936 x 4096 (packed tiles from batch 8, GGUF rows below); a batch of sequences
    with contexts U[256, 8192]."""
    from rta import model, ops
    batch = args.batch or 32
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(20261110 + 5)
    ctx = rng.integers(256, 8193, batch).astype(np.int32)
    capacity = 8192 + 256
    # the weight layout each batch runs fastest on (measured): packed tiles on the matrix
    # cores from 8 rows up, GGUF rows on the batch-1 vector-ALU readouts below (--packed:
    # packed tiles at any batch, for the comparison)
    packed = batch >= 8 or args.packed
    shape = model.shape_9b(capacity, packed=packed)
    want_cpu = not args.no_cpu and batch == 32
    m = model.DecodeModel(shape, batch, ctx, seed=20261115, keep_gguf=want_cpu)
    nfull = shape.layers // shape.full_every
    nrec = shape.layers - nfull
    # decode attention of the batch over one full-attention layer's history, rotated over
    # the 8 layers' distinct histories (8 x 383 MB)
    v = m.views
    per_layer = v.slots_per_layer * v.packet_bytes
    p0 = v.packets - m.state.data_ptr()
    hist_layers = [m.state[p0 + l * per_layer:p0 + (l + 1) * per_layer] for l in range(nfull)]
    hq, hkv, hd = shape.q_heads, shape.kv_heads, shape.head_dim
    qa = torch.randn(batch, hq, hd, device=dev)
    oa = torch.empty_like(qa)
    base = torch.arange(batch, dtype=torch.int64, device=dev) * capacity
    ctx_d = torch.from_numpy(ctx).to(dev)
    aws = torch.empty(ops.decode_attention_workspace_bytes(batch, hq, hkv, hd, capacity), dtype=torch.uint8,
                      device=dev)

    def step(i):
        m.step()

    def attention(i):
        ops.decode_attention(qa, hist_layers[i % nfull], shape.fmt_k, shape.fmt_v, base, ctx_d, capacity, capacity,
                             hkv, workspace=aws, out=oa)

    # the LM head (510 MB, two copies rotate past the cache)
    lm2 = model.random_kquant(Q6_K, shape.vocab, shape.hidden, torch.Generator(device=dev), dev)
    lm_copies = [m.lm_head, ops.pack(Q6_K, lm2, shape.vocab, shape.hidden) if packed else lm2]
    hn = torch.randn(batch, shape.hidden, device=dev)
    lg = torch.empty(batch, shape.vocab, device=dev)
    ids = torch.empty(batch, dtype=torch.int32, device=dev)
    lws = torch.empty(ops.lm_head_workspace_bytes(shape.fmt_lm, shape.vocab, shape.hidden, batch),
                      dtype=torch.uint8, device=dev)

    def lm_head(i):
        ops.lm_head(shape.fmt_lm, lm_copies[i % 2], shape.vocab, shape.hidden, hn, workspace=lws, logits=lg, ids=ids)

    w_bytes = m.weight_bytes() - m.lm_head.numel()                       # projections + small vectors
    sum_ctx = int(sum(min(int(c), capacity) for c in ctx))
    hist = sum_ctx * nfull * v.packet_bytes                             # history read per step (approx.)
    state = 2 * nrec * batch * shape.rec_heads * 128 * 128 * 4          # recurrent state read + write
    step_bytes = w_bytes + m.lm_head.numel() + hist + state
    kernels = step_kernels(torch, shape, batch, dev, packed)
    kernels.append((f"attention: attn_qprep_kernel + attn_chunk_mma_kernel<G=4,KPW=2> + attn_merge_kernel ({batch} "
                    f"sequences, {hq}/{hkv} heads, {sum_ctx} positions of {v.packet_bytes}-byte packets)", nfull,
                    sum_ctx * v.packet_bytes + 2 * batch * hq * hd * 4, attention))
    kernels.append((f"LM head: {'gemm_tiled_kernel' if packed else 'gemv_b1_kernel'}<Q6_K,logits> + group max + "
                    f"argmax_margin_kernel (rta_lm_head, {'packed' if packed else 'GGUF rows'} 151936x4096)", 1, m.lm_head.numel() + 4 * batch * (shape.hidden + shape.vocab), lm_head))
    # HBM bytes measured per launch at this batch (the batch-32 figures under "decode/...")
    res = {"alg_bytes": step_bytes, "graph_per_step": True, "kernels": kernels,
           "traffic_prefix": "decode" if batch == 32 else f"decode_b{batch}",
           "step": step, "unit": "tok/s", "value_from_ms": lambda ms: batch / (ms * 1e-3),
           "dtype": "q4_k/q6_k weights x fp32 activations and state, fp32 accumulate",
           "config": {"workload": f"9B-shape hybrid decode step, batch {batch} (32 layers: 24 gated delta-net + 8 "
                                  "full attention; hidden 4096, 32/8 heads x 128, FF 12288, Q4_K projections, "
                                  "Q6_K LM head 151936x4096; contexts U[256, 8192], greedy)",
                      "weight_layout": "packed tiles" if packed else "GGUF rows",
                      "batch": batch, "layers": 32, "hidden": 4096, "ff": 12288, "vocab": 151936,
                      "sum_context": int(ctx.sum()), "history_capacity": capacity,
                      "bytes_per_step": int(step_bytes), "weight_bytes_per_step": int(w_bytes + m.lm_head.numel()),
                      "seed": "20261110+5"}}
    snap = {}

    def check():
        # the state before this step, for the CPU step that runs from the same point
        if want_cpu:
            snap.update(rec=np.ascontiguousarray(m.state_view("recurrent")),
                        conv=np.ascontiguousarray(m.state_view("conv")),
                        packets=np.ascontiguousarray(m.state_view("packets")), ctx=m.state_view("ctx"),
                        tokens=m.tokens.cpu().numpy().view(np.uint32).copy())
        m.step(logits=True)
        lgt = m.logits.cpu().numpy()
        toks = m.tokens.cpu().numpy().view(np.uint32)
        snap.update(gpu_logits=lgt.copy(), gpu_tokens=toks.copy())
        ok = bool(np.isfinite(lgt).all()) and all(int(toks[b]) == orc.argmax_margin_f32(lgt[b], 1e-4)
                                                  for b in range(batch))
        return {"tokens_follow_margin_rule": ok, "logits_finite": bool(np.isfinite(lgt).all()), "ok": ok,
                "note": "the 9B step at 4 layers against the fp64 composition: tests/test_gpu_sizes.py; "
                        "cpu_baseline.parity: this step against the fp32 CPU step from the same state"}

    def cpu(seconds):
        t = omp_threads()
        cs = orc.CpuStep(shape, m.gguf)
        st = {k: snap[k].copy() for k in ("rec", "conv", "packets", "ctx", "tokens")}
        lg_cpu = np.empty((batch, shape.vocab), np.float32)
        n, t0 = 0, time.perf_counter()
        while True:
            cs.step(batch, st["rec"], st["conv"], st["packets"], st["ctx"], st["tokens"],
                    lg_cpu if n == 0 else None, threads=t)
            if n == 0:
                par = close(snap["gpu_logits"], lg_cpu)
                same = int(np.sum(st["tokens"] == snap["gpu_tokens"]))
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        return {"value": batch * n / el, "unit": "tok/s", "cores": t, "kind": "port",
                "sample": f"{n} whole decode step(s) of the 9B shape at batch {batch} (all 32 layers, LM head and "
                          f"argmax) by the oracle's fp32 OpenMP CPU step (oracle/rta_cpu_step.c, -O3 AVX2/FMA) "
                          f"in {el:.1f} s on {t} threads of {cpu_model()}",
                "parity": {"logits_vs_gpu_step": par, "tokens_equal": f"{same}/{batch}"}}
    res["check"], res["cpu"] = check, cpu
    return res


def w_copy_calib(torch, args, orc):
    dev = torch.device("cuda:0")
    n = 64 << 20
    src = [torch.empty(n, dtype=torch.uint8, device=dev).fill_(1) for _ in range(14)]
    dst = torch.empty(n, dtype=torch.uint8, device=dev)

    def step(i):
        dst.copy_(src[i % len(src)])

    res = {"alg_bytes": 2 * n, "kernel": "device-to-device copy of 64 MiB", "step": step, "kernel_launch": step,
           "unit": "GB/s", "value_from_ms": lambda ms: 2 * n / (ms * 1e-3) / 1e9, "dtype": "u8",
           "config": {"workload": "plain copy 64 MiB (read 64 MiB + write 64 MiB), PMC calibration"},
           "check": lambda: {"ok": True}, "cpu": None}
    return res


def companions(torch, args, orc):
    """The metric's other two figures, measured in the same run as the batch-32 decode step:
    the same step at batch 1 (tok/s) and the single Q4_K GEMV 4096x4096 (GB/s, HBM fraction)."""
    import argparse as ap
    a1 = ap.Namespace(**vars(args))
    a1.batch = 1
    d1 = w_decode(torch, a1, orc)
    p1 = d1["check"]()
    ms1 = timed_replays(torch, d1["step"], args.steps, args.warmup) / args.steps
    out = {"decode_batch1": {"value": d1["value_from_ms"](ms1), "unit": "tok/s", "ms_per_step": ms1,
                             "steps": args.steps, "parity": p1, "config": d1["config"]}}
    del d1
    g = w_gemv_q4k(torch, args, orc)
    pg = g["check"]()
    k = time_kernel(torch, g["kernel_launch"])
    ms = timed_region(torch, g["step"], 1000, 100) / 1000
    gbs = g["value_from_ms"](ms)
    ach = g["alg_bytes"] / (k * 1e-3) / 1e9
    out["gemv_q4k"] = {"value": gbs, "unit": "GB/s", "steps": 1000, "ms_per_step": ms, "frac_of_hbm_peak":
                       gbs / HBM_PEAK_GBS, "roofline": {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS,
                                                       "unit": "GB/s", "frac": ach / HBM_PEAK_GBS,
                                                       "traffic": traffic_for("gemv_q4k")},
                       "kernel": g["kernel"], "kernel_ms_mean": k, "parity": pg, "config": g["config"]}
    at = read_ceiling_at(torch, g["alg_bytes"])
    if at:
        out["gemv_q4k"]["read_ceiling_at_size"] = at
        out["gemv_q4k"]["roofline"]["frac_of_size_ceiling"] = ach / at["gbs"]
    return out


WORKLOADS = {"gemv_q4k": w_gemv_q4k, "mlp": w_mlp, "lm_head": w_lm_head, "attention": w_attention,
             "proj": w_proj, "decode": w_decode, "copy_calib": w_copy_calib}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 (no multi-GPU path is "
                                   "built: every GPU box here has one GPU)"}))
        sys.exit(2)
    import torch
    from rta import _lib
    _lib.load()
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as orc
    if args.steps is None:
        args.steps = 64 if args.workload == "decode" else 1000
    if args.warmup is None:
        args.warmup = 4 if args.workload == "decode" else 100
    wl = WORKLOADS[args.workload](torch, args, orc)
    parity = wl["check"]()
    if wl.get("graph_per_step") and not args.eager:
        ms = timed_replays(torch, wl["step"], args.steps, args.warmup)
    else:
        ms = timed_region(torch, wl["step"], args.steps, args.warmup, args.eager)
    ms_step = ms / args.steps
    # the dominant kernel: the one with the largest share of a step (calls per step x mean
    # duration) when the workload lists several, else the workload's own
    table = []
    for name, calls, alg, launch in wl.get("kernels", []):
        km = time_kernel(torch, launch)
        ach = alg / (km * 1e-3) / 1e9
        key = f"{wl.get('traffic_prefix', args.workload)}/{name.split(':')[0]}"
        table.append({"kernel": name, "calls_per_step": calls, "ms_mean": km, "alg_bytes": alg,
                      "achieved_gbs": ach, "frac": ach / HBM_PEAK_GBS, "ms_per_step": calls * km,
                      "traffic": traffic_for(key)})
    if table:
        dom = max(table, key=lambda r: r["ms_per_step"])
        kernel_name, k_mean, alg_k, traffic = dom["kernel"], dom["ms_mean"], dom["alg_bytes"], dom["traffic"]
    else:
        k_mean = time_kernel(torch, wl["kernel_launch"])
        kernel_name, alg_k = wl["kernel"], wl.get("alg_bytes_kernel", wl["alg_bytes"])
        traffic = traffic_for(args.workload)
    achieved = alg_k / (k_mean * 1e-3) / 1e9
    cpu = None if (args.no_cpu or wl["cpu"] is None) else wl["cpu"](args.cpu_seconds)
    line = {"metric": METRIC, "value": wl["value_from_ms"](ms_step), "unit": wl["unit"], "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": wl["dtype"], "data": "synthetic",
            "timing": "eager launches" if args.eager else ("one HIP graph of a step, replayed per step"
                                                            if wl.get("graph_per_step") else
                                                            "one HIP graph replay of all steps"),
            "config": wl["config"],
            "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": achieved / HBM_PEAK_GBS, "traffic": traffic},
            "cpu_baseline": cpu, "kernel": kernel_name, "kernel_ms_mean": k_mean,
            "alg_bytes_per_launch": alg_k, "alg_bytes_per_step": wl["alg_bytes"], "parity": parity}
    if table:
        line["kernels"] = table
    ceil = read_ceiling(torch)
    if ceil:
        line["read_ceiling"] = ceil
        line["roofline"]["ceiling"] = ceil["gbs"]
        line["roofline"]["frac_of_ceiling"] = achieved / ceil["gbs"]
    if args.workload == "gemv_q4k":
        at = read_ceiling_at(torch, alg_k)
        if at:
            line["read_ceiling_at_size"] = at
            line["roofline"]["frac_of_size_ceiling"] = achieved / at["gbs"]
    if args.workload == "decode" and not args.no_companions:
        line["companions"] = companions(torch, args, orc)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
