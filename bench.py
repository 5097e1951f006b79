#!/usr/bin/env python3
"""Benchmark of the Q4 decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line.  Workloads (inputs synthetic, seeded, generated in HBM
before the timed region; weights rotate over enough distinct copies that the
working set exceeds the 256 MB Infinity Cache, so every step streams HBM):

  mlp   (default) fused Q4 gated MLP decode step at 12B dims: hidden 3840,
        FFN 15360: fused gate/up + GELU-tanh (chn_fused_mlp_q4), then down
        (chn_gemv_q4).  One step = one token's MLP.
  gemv  single Q4 matvec, W 8192 x 2048, x fp32 [2048].

`roofline` is for the dominant kernel (the fused gate/up matvec for `mlp`),
timed with HIP events on the library's stream over back-to-back launches;
`cpu_baseline` times the oracle's threaded restatement of the same step on
this host's cores (rank 0, N=1 only) on a bounded sample.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
METRIC = "decode tok/s + Q4 GEMV achieved HBM GB/s (% of peak), 12B-class, 1 GPU"
SEED = 0xC4A77E1
ROTATE_BYTES = 1 << 30  # >= 4x the 256 MB Infinity Cache


def q4_bytes(rows, K):
    return rows * (K // 32) * 20


def load_traffic(kernel, workload):
    """HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE, from profiles/traffic.md (None if not measured)."""
    path = os.path.join(ROOT, "profiles", "traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 6 and cells[0] == kernel and cells[1] == workload:
            try:
                return float(cells[5])
            except ValueError:
                return None
    return None


def cpu_info():
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return n, model


def bench_mlp(ctx, args):
    import numpy as np

    H, I = 3840, 15360
    w_bytes = q4_bytes(I, H)
    ncopy = max(4, -(-ROTATE_BYTES // (3 * w_bytes)))
    Wg, Wu, Wd = [], [], []
    for c in range(ncopy):
        for lst, rows, K, k in ((Wg, I, H, 0), (Wu, I, H, 1), (Wd, H, I, 2)):
            b = ctx.alloc(q4_bytes(rows, K))
            ctx.call("chn_synth_q4", b, rows, K, SEED + 16 * c + k, 0.005, 0.02)
            lst.append(b)
    x = ctx.alloc(H * 4)
    ctx.call("chn_synth_normal", x, H, SEED + 7, 1.0)
    act = ctx.alloc(I * 4)
    y = ctx.alloc(H * 4)
    ctx.sync()

    def step(i):
        c = i % ncopy
        ctx.call("chn_fused_mlp_q4", Wg[c], Wu[c], x, act, I, H)
        ctx.call("chn_gemv_q4", Wd[c], act, y, H, I)

    for i in range(args.warmup):
        step(i)
    ctx.sync()
    t0 = time.perf_counter()
    ctx.timer_start()
    for i in range(args.steps):
        step(i)
    gpu_ms = ctx.timer_stop()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms_per_step = max(gpu_ms, wall_ms) / args.steps

    # dominant kernel alone, back to back on the same stream
    reps = max(args.steps, 64)
    ctx.timer_start()
    for i in range(reps):
        c = i % ncopy
        ctx.call("chn_fused_mlp_q4", Wg[c], Wu[c], x, act, I, H)
    k_ms = ctx.timer_stop() / reps
    ctx.timer_start()
    for i in range(reps):
        c = i % ncopy
        ctx.call("chn_gemv_q4", Wd[c], act, y, H, I)
    d_ms = ctx.timer_stop() / reps

    step_bytes = 3 * w_bytes + H * 4 + H * 4 + 2 * I * 4
    gateup_bytes = 2 * w_bytes + H * 4 + I * 4
    down_bytes = w_bytes + I * 4 + H * 4
    achieved = gateup_bytes / (k_ms * 1e-3) / 1e9
    traffic = load_traffic("k_matvec_q4<MLP>", "mlp")

    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        nthr, model = cpu_info()
        hg = ctx.download(Wg[0], np.uint32, w_bytes // 4)
        hu = ctx.download(Wu[0], np.uint32, w_bytes // 4)
        hd = ctx.download(Wd[0], np.uint32, w_bytes // 4)
        hx = ctx.download(x, np.float32, H)
        n, t_start = 0, time.perf_counter()
        while True:
            oracle.fused_mlp_step_mt(hg, hu, hd, hx, H, I, nthr - 1)
            n += 1
            if time.perf_counter() - t_start >= args.cpu_seconds:
                break
        dt = time.perf_counter() - t_start
        cpu = {"value": n / dt, "unit": "steps/s", "cores": nthr, "kind": "port",
               "sample": f"{n} MLP decode steps (gate/up 15360x3840 + down 3840x15360 Q4), "
                         f"{nthr} threads ({nthr - 1} pool workers + caller), {model}"}

    return {
        "value": 1e3 / ms_per_step,
        "unit": "MLP decode steps/s",
        "ms_per_step": ms_per_step,
        "config": {"workload": "fused Q4 gated MLP decode step (gate/up/down Q4, GELU-tanh)",
                   "hidden": H, "ffn": I, "batch": 1, "weight_copies_rotated": ncopy,
                   "step_hbm_gbps": step_bytes / (ms_per_step * 1e-3) / 1e9,
                   "step_bytes": step_bytes,
                   "down_gemv_ms": d_ms,
                   "down_gemv_gbps": down_bytes / (d_ms * 1e-3) / 1e9},
        "roofline": {"kernel": "k_matvec_q4<MLP> (fused gate/up + GELU-tanh)",
                     "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "algorithmic_bytes_per_launch": gateup_bytes,
                     "avg_launch_ms": k_ms},
        "cpu_baseline": cpu,
        "dtype": "fp32 accumulate over Q4 weights",
    }


def bench_gemv(ctx, args):
    import numpy as np

    M, K = 8192, 2048
    w_bytes = q4_bytes(M, K)
    ncopy = max(32, -(-ROTATE_BYTES // w_bytes))
    Ws = []
    for c in range(ncopy):
        b = ctx.alloc(w_bytes)
        ctx.call("chn_synth_q4", b, M, K, SEED + c, 0.005, 0.02)
        Ws.append(b)
    x = ctx.alloc(K * 4)
    ctx.call("chn_synth_normal", x, K, SEED + 999, 1.0)
    y = ctx.alloc(M * 4)
    ctx.sync()
    for i in range(args.warmup):
        ctx.call("chn_gemv_q4", Ws[i % ncopy], x, y, M, K)
    ctx.sync()
    t0 = time.perf_counter()
    ctx.timer_start()
    for i in range(args.steps):
        ctx.call("chn_gemv_q4", Ws[i % ncopy], x, y, M, K)
    gpu_ms = ctx.timer_stop()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms = max(gpu_ms, wall_ms) / args.steps
    k_ms = gpu_ms / args.steps
    nbytes = w_bytes + K * 4 + M * 4
    achieved = nbytes / (k_ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        nthr, model = cpu_info()
        hw = ctx.download(Ws[0], np.uint32, w_bytes // 4)
        hx = ctx.download(x, np.float32, K)
        n, t_start = 0, time.perf_counter()
        while True:
            oracle.gemv_q4_mt(hw, hx, M, K, nthr - 1)
            n += 1
            if time.perf_counter() - t_start >= args.cpu_seconds:
                break
        dt = time.perf_counter() - t_start
        cpu = {"value": n / dt, "unit": "GEMV/s", "cores": nthr, "kind": "port",
               "sample": f"{n} Q4 GEMVs 8192x2048, {nthr} threads, {model}"}
    return {
        "value": 1e3 / ms, "unit": "GEMV/s", "ms_per_step": ms,
        "config": {"workload": "single Q4 matvec 8192x2048", "M": M, "K": K, "batch": 1,
                   "weight_copies_rotated": ncopy},
        "roofline": {"kernel": "k_matvec_q4<GEMV>", "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": load_traffic("k_matvec_q4<GEMV>", "gemv"),
                     "algorithmic_bytes_per_launch": nbytes, "avg_launch_ms": k_ms},
        "cpu_baseline": cpu,
        "dtype": "fp32 accumulate over Q4 weights",
    }


def bench_prefill(ctx, args):
    """Batched prefill Q4 GEMM: 512 tokens x K=3840 -> 15360 features."""
    T, K, N = 512, 3840, 15360
    w_bytes = q4_bytes(N, K)
    ncopy = 4
    Ws = []
    for c in range(ncopy):
        b = ctx.alloc(w_bytes)
        ctx.call("chn_synth_q4", b, N, K, SEED + c, 0.005, 0.02)
        Ws.append(b)
    X = ctx.alloc(T * K * 4)
    ctx.call("chn_synth_normal", X, T * K, SEED + 77, 1.0)
    Y = ctx.alloc(T * N * 4)
    ctx.sync()
    for i in range(args.warmup):
        ctx.call("chn_batch_gemm_q4", Ws[i % ncopy], X, Y, T, N, K)
    ctx.sync()
    t0 = time.perf_counter()
    ctx.timer_start()
    for i in range(args.steps):
        ctx.call("chn_batch_gemm_q4", Ws[i % ncopy], X, Y, T, N, K)
    gpu_ms = ctx.timer_stop()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms = max(gpu_ms, wall_ms) / args.steps
    flops = 2.0 * T * K * N
    achieved = flops / (gpu_ms / args.steps * 1e-3) / 1e12
    return {
        "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms,
        "config": {"workload": "batched prefill Q4 GEMM 512 tokens x 3840 -> 15360 (bf16 MFMA)",
                   "tokens": T, "K": K, "N": N, "flop_per_step": flops},
        "roofline": {"kernel": "k_q4gemm<1> (+ k_to_bf16 pre-pass)", "bound": "mfma",
                     "achieved": achieved, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / MFMA_BF16_PEAK_TFLOPS, "traffic": None,
                     "algorithmic_flop_per_launch": flops,
                     "avg_launch_ms": gpu_ms / args.steps},
        "cpu_baseline": None,
        "dtype": "bf16 MFMA operands, fp32 accumulate",
    }


def bench_attn(ctx, args):
    """Decode attention, 16 query / 8 KV heads, head_dim 256, full 4096-slot
    ring of fp32 K/V."""
    import numpy as np

    H, KVH, D, S = 16, 8, 256, 4096
    kv_dim = KVH * D
    ncopy = 4     # 4 x 67 MB caches > 256 MB Infinity Cache
    Kc, Vc = [], []
    for c in range(ncopy):
        k = ctx.alloc(S * kv_dim * 4)
        v = ctx.alloc(S * kv_dim * 4)
        ctx.call("chn_synth_normal", k, S * kv_dim, SEED + 100 + c, 1.0)
        ctx.call("chn_synth_normal", v, S * kv_dim, SEED + 200 + c, 1.0)
        Kc.append(k)
        Vc.append(v)
    q = ctx.alloc(H * D * 4)
    ctx.call("chn_synth_normal", q, H * D, SEED + 300, 0.1)
    slots = ctx.upload(((np.arange(S) + 1234) % S).astype(np.uint32))
    ns = ctx.upload(np.array([S], np.uint32))
    out = ctx.alloc(H * D * 4)
    ctx.sync()
    for i in range(args.warmup):
        ctx.call("chn_decode_attn", q, Kc[i % ncopy], Vc[i % ncopy], slots, ns, S, H, D, kv_dim, 2, 1.0, out)
    ctx.sync()
    t0 = time.perf_counter()
    ctx.timer_start()
    for i in range(args.steps):
        ctx.call("chn_decode_attn", q, Kc[i % ncopy], Vc[i % ncopy], slots, ns, S, H, D, kv_dim, 2, 1.0, out)
    gpu_ms = ctx.timer_stop()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms = max(gpu_ms, wall_ms) / args.steps
    nbytes = 2 * S * kv_dim * 4 + S * 4 + 2 * H * D * 4
    achieved = nbytes / (gpu_ms / args.steps * 1e-3) / 1e9
    return {
        "value": 1e3 / ms, "unit": "attention steps/s", "ms_per_step": ms,
        "config": {"workload": "decode attention over a full 4096-slot ring (16 q / 8 kv heads, D 256)",
                   "slots": S, "bytes_per_step": nbytes},
        "roofline": {"kernel": "k_attn_split + k_attn_combine", "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": None, "algorithmic_bytes_per_launch": nbytes,
                     "avg_launch_ms": gpu_ms / args.steps},
        "cpu_baseline": None,
        "dtype": "fp32",
    }


WORKLOADS = {"mlp": bench_mlp, "gemv": bench_gemv, "prefill": bench_prefill, "attn": bench_attn}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="mlp", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures the single-GPU hot path only: run it with --gpus 1 "
              "(this build has no multi-GPU path; see DESIGN.md for how it would shard).",
              file=sys.stderr)
        sys.exit(2)

    import __graft_entry__
    __graft_entry__._ensure_built()
    import channel_amd as ca

    with ca.Context(0) as ctx:
        r = WORKLOADS[args.workload](ctx, args)
    line = {
        "metric": METRIC,
        "value": r["value"],
        "unit": r["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": r["dtype"],
        "data": "synthetic (seeded; Q4 codes uniform 0..15, f16 scales U(0.005, 0.02), "
                "x ~ N(0,1))",
        "config": r["config"],
        "roofline": r["roofline"],
        "cpu_baseline": r["cpu_baseline"],
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
