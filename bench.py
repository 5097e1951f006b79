#!/usr/bin/env python3
"""Benchmark of the Q4 decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line.  Workloads (inputs synthetic, seeded, generated in HBM
before the timed region; weights rotate over enough distinct copies that the
working set exceeds the 256 MB Infinity Cache, so every step streams HBM):

  decode  (default) the full 48-layer 12B-class Q4 model (hidden 3840, FFN
          15360, 16 query / 8 KV heads, head_dim 256, vocab 262144, every
          fifth layer global, sliding window 512): a 512-token prompt of
          uniform random ids is prefilled, then greedy decode steps run
          through the recorded decode graph.  One step = one token
          (embedding gather, 48 layers, Q8 logits, top-64, argmax).
  mlp     fused Q4 gated MLP decode step at 12B dims: fused gate/up +
          GELU-tanh (chn_fused_mlp_q4), then down (chn_gemv_q4).
  gemv    single Q4 matvec, W 8192 x 2048, x fp32 [2048].
  prefill batched prefill Q4 GEMM 512 x 3840 -> 15360 on bf16 MFMA.
  attn    decode attention over a full 4096-slot ring.

`roofline` is for the dominant kernel (the fused gate/up matvec for decode
and mlp), timed with HIP events on the library's stream over back-to-back
launches; `cpu_baseline` times the oracle's threaded restatement of the same
work on this host's cores (rank 0, N=1 only) on a bounded sample.
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
# What the decode matvecs compute in: Q4 weights times activations rounded
# to 18-bit block fixed point (per 32-block, 2^-18 of the block's power-of-
# two bound), exact int32 block dots, fp32 across blocks.
DTYPE_Q4MV = ("q4 x 18-bit block-fixed-point activations (exact int32 block dots via v_dot8c_i32_i4, "
              "fp32 across blocks)")
DTYPE_DECODE = (DTYPE_Q4MV + "; q8 logits x 22-bit block-fixed-point activations; fp32 attention, norms and "
                "KV cache")


def q4_bytes(rows, K):
    return rows * (K // 32) * 20


def xplanes_bytes(K):
    return (K // 32) * 21 * 4


def q4r_bytes(rows, K):
    return rows * (K // 32) * 18


def load_traffic(kernel, workload):
    """HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE and calibrated on a plain copy, read from the table in
    profiles/traffic.md (None if that kernel and workload were not measured)."""
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
    rep = args.layout == "q4r"
    w_bytes = q4_bytes(I, H)               # algorithmic bytes (the reference layout)
    ncopy = max(4, -(-ROTATE_BYTES // (3 * w_bytes)))
    mlp_fn, gemv_fn = "chn_fused_mlp_q4", "chn_gemv_q4"     # repacked: replaced below
    Wg, Wu, Wd = [], [], []
    ref0 = []                              # copy 0 in the reference layout, for the CPU baseline
    for c in range(ncopy):
        for lst, rows, K, k in ((Wg, I, H, 0), (Wu, I, H, 1), (Wd, H, I, 2)):
            b = ctx.alloc(q4_bytes(rows, K))
            ctx.call("chn_synth_q4", b, rows, K, SEED + 16 * c + k, 0.005, 0.02)
            if rep:
                r = ctx.alloc(q4r_bytes(rows, K))
                ctx.call("chn_q4_repack", b, rows, K, r)
                ctx.sync()
                if c == 0:
                    ref0.append(b)
                else:
                    b.free()
                b = r
            elif c == 0:
                ref0.append(b)
            lst.append(b)
    x = ctx.alloc(H * 4)
    ctx.call("chn_synth_normal", x, H, SEED + 7, 1.0)
    act = ctx.alloc(I * 4)
    y = ctx.alloc(H * 4)
    if rep:
        # as the model runs it: planes of x once (the norm kernel writes them
        # there), gate/up writing act and its planes, down reading those
        xpl, apl = ctx.alloc(xplanes_bytes(H)), ctx.alloc(xplanes_bytes(I))
        ctx.call("chn_xplanes", x, H, xpl)
        mlp_fn, gemv_fn = "chn_fused_mlp_q4r_xp", "chn_gemv_q4r_xp"
        mlp_args = lambda c: (Wg[c], Wu[c], xpl, act, apl, I, H)
        gemv_args = lambda c: (Wd[c], apl, y, H, I)
    else:
        mlp_args = lambda c: (Wg[c], Wu[c], x, act, I, H)
        gemv_args = lambda c: (Wd[c], act, y, H, I)
    ctx.sync()

    mlp_calls = [ctx.bind(mlp_fn, *mlp_args(c)) for c in range(ncopy)]
    gemv_calls = [ctx.bind(gemv_fn, *gemv_args(c)) for c in range(ncopy)]

    def step(i):
        mlp_calls[i % ncopy]()
        gemv_calls[i % ncopy]()

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
        mlp_calls[i % ncopy]()
    k_ms = ctx.timer_stop() / reps
    ctx.timer_start()
    for i in range(reps):
        gemv_calls[i % ncopy]()
    d_ms = ctx.timer_stop() / reps

    step_bytes = 3 * w_bytes + H * 4 + H * 4 + 2 * I * 4
    gateup_bytes = 2 * w_bytes + H * 4 + I * 4
    down_bytes = w_bytes + I * 4 + H * 4
    achieved = gateup_bytes / (k_ms * 1e-3) / 1e9
    traffic = load_traffic("k_q4rmv_mlp_xp" if rep else "k_q4mv<MLP>", "gate/up 15360x3840")

    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        nthr, model = cpu_info()
        hg, hu, hd = (ctx.download(b, np.uint32, w_bytes // 4) for b in ref0)
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
                   "weight_layout": "repacked Q4R (18 B per 32 weights)" if rep else "reference Q4 (20 B)",
                   "step_hbm_gbps": step_bytes / (ms_per_step * 1e-3) / 1e9,
                   "step_bytes": step_bytes,
                   "down_gemv_ms": d_ms,
                   "down_gemv_gbps": down_bytes / (d_ms * 1e-3) / 1e9},
        "roofline": {"kernel": ("k_q4rmv_mlp_xp (chn_fused_mlp_q4r_xp: gate/up + GELU-tanh + planes of act)" if rep
                                else "chn_fused_mlp_q4 = k_xplanes + k_q4mv<MLP> (fused gate/up + GELU-tanh)"),
                     "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "algorithmic_bytes_per_launch": gateup_bytes,
                     "avg_launch_ms": k_ms},
        "cpu_baseline": cpu,
        "dtype": DTYPE_Q4MV if rep else DTYPE_Q4MV + " (reference layout)",
    }


def alloc_gateup_copies(ctx, H, I, min_bytes=ROTATE_BYTES, repacked=False):
    """Distinct 12B-dims gate/up pairs, enough to exceed the Infinity Cache,
    in the reference Q4 layout or repacked (Q4R, the model's layout)."""
    w_bytes = q4_bytes(I, H)
    ncopy = max(4, -(-min_bytes // (2 * w_bytes)))
    pairs = []
    for c in range(ncopy):
        pair = []
        for k in range(2):
            w = ctx.alloc(w_bytes)
            ctx.call("chn_synth_q4", w, I, H, SEED + 16 * c + k, 0.005, 0.02)
            if repacked:
                r = ctx.alloc(q4r_bytes(I, H))
                ctx.call("chn_q4_repack", w, I, H, r)
                ctx.sync()
                w.free()
                w = r
            pair.append(w)
        pairs.append(tuple(pair))
    return pairs


def time_gateup(ctx, pairs, x, act, H, I, reps, repacked=False, fused_norm=False):
    """Average duration (ms) of the fused gate/up matvec over back-to-back
    launches on the library stream, HIP events.  fused_norm: the decode
    step's launch (chn_ffn_gate_up_q4r = k_q4rmv_mlp_xp<8, NORM_POST_ADD>:
    post-attention norm, residual add and pre-FFN norm as the prologue,
    act and its planes out); repacked: the same matvec reading ready-made
    planes of x (k_q4rmv_mlp_xp<4, -1>, x's planes made once beforehand);
    reference layout: chn_fused_mlp_q4 (its planes pass + matvec)."""
    if fused_norm:
        r = ctx.alloc(H * 4)
        ctx.call("chn_synth_normal", r, H, SEED + 8, 1.0)
        ones = ctx.alloc(H * 4)
        ctx.fill_u32(ones, 0x3F800000, H)
        x_out, normed = ctx.alloc(H * 4), ctx.alloc(H * 4)
        act_planes = ctx.alloc(xplanes_bytes(I))
        calls = [ctx.bind("chn_ffn_gate_up_q4r", g, u, x, r, ones, ones, x_out, normed, act, act_planes, I, H, 1e-6)
                 for g, u in pairs]
    elif repacked:
        planes = ctx.alloc(xplanes_bytes(H))
        act_planes = ctx.alloc(xplanes_bytes(I))
        ctx.call("chn_xplanes", x, H, planes)
        calls = [ctx.bind("chn_fused_mlp_q4r_xp", g, u, planes, act, act_planes, I, H) for g, u in pairs]
    else:
        calls = [ctx.bind("chn_fused_mlp_q4", g, u, x, act, I, H) for g, u in pairs]
    for i in range(4):
        calls[i % len(calls)]()
    ctx.timer_start()
    for i in range(reps):
        calls[i % len(calls)]()
    return ctx.timer_stop() / reps


def gateup_bytes(H, I, repacked=False, fused_norm=False):
    """Bytes of one gate/up launch: the reference layout's algorithmic count
    (20 B per 32 weights), or what the repacked layout reads (18 B); x in,
    act out.  fused_norm: the decode step's form also reads x_in, r and the
    two norm weights, writes x_out and the planes of act (84 B per 32)."""
    w = q4r_bytes(I, H) if repacked else q4_bytes(I, H)
    if fused_norm:
        return 2 * w + 5 * H * 4 + I * 4 + xplanes_bytes(I)
    return 2 * w + H * 4 + I * 4


CFG_12B = dict(hidden_size=3840, intermediate_size=15360, vocab_size=262144, num_layers=48,
               num_heads=16, num_kv_heads=8, head_dim=256, rotary_dim=256, rms_norm_eps=1e-6,
               rope_theta=1e4, rope_theta_full=1e6, sliding_window=512, k_eq_v=0,
               max_prefill_tokens=512, layer_full=[1 if (l + 1) % 5 == 0 else 0 for l in range(48)])
PROMPT = 512


def token_bytes(cfg, ctx_len):
    """Algorithmic HBM bytes of one decode token: every Q4 layer matrix and
    the Q8 tied embedding once, plus the K/V rows each layer's attention
    reads (fp32) and the new K/V row it writes."""
    H, I, D = cfg["hidden_size"], cfg["intermediate_size"], cfg["head_dim"]
    qd, kvd = cfg["num_heads"] * D, cfg["num_kv_heads"] * D
    layer_w = q4_bytes(qd + 2 * kvd, H) + q4_bytes(H, qd) + 2 * q4_bytes(I, H) + q4_bytes(H, I)
    w = cfg["num_layers"] * layer_w + cfg["vocab_size"] * (H // 32) * 36
    kv = 0
    for full in cfg["layer_full"]:
        n = ctx_len if full else min(ctx_len, cfg["sliding_window"])
        kv += 2 * n * kvd * 4 + 2 * kvd * 4
    return w, kv


def cpu_decode_sample(cfg, seed, ctx_len, seconds):
    """The oracle's threaded restatement of one decode token, timed on a
    bounded sample: two layers (one sliding, one global) with the synthetic
    model's own seeded weights, stepped alternately for about `seconds`, and
    the Q8 logits over a 16384-row slice of the vocabulary plus one top-64
    over 262144 logits; scaled to a 48-layer, 262144-vocab token."""
    import numpy as np

    import oracle
    nthr, model = cpu_info()
    nthr = min(nthr, 16)
    H, I, D = cfg["hidden_size"], cfg["intermediate_size"], cfg["head_dim"]
    nq, nkv = cfg["num_heads"], cfg["num_kv_heads"]
    qd, kvd = nq * D, nkv * D
    eps = cfg["rms_norm_eps"]
    layers = []
    for li in (0, 4):
        ls = seed + 64 * (li + 1)
        shapes = [(qd, H), (kvd, H), (kvd, H), (H, qd), (I, H), (I, H), (H, I)]
        W = [oracle.synth_q4(r, k, ls + j) for j, (r, k) in enumerate(shapes)]
        layers.append((li, W))
    kc = oracle.synth_normal(4096 * kvd, seed + 11)
    vc = oracle.synth_normal(4096 * kvd, seed + 12)
    ones_h = np.ones(H, np.float32)
    ones_d = np.ones(D, np.float32)
    x = oracle.synth_normal(H, seed + 13)
    slots_full = np.arange(ctx_len, dtype=np.uint32)
    slots_sl = slots_full[-cfg["sliding_window"]:]

    def layer_step(li, W, x):
        full = cfg["layer_full"][li]
        normed = oracle.rmsnorm(x, ones_h, eps)
        q = oracle.gemv_q4_mt(W[0], normed, qd, H, nthr - 1)
        k = oracle.gemv_q4_mt(W[1], normed, kvd, H, nthr - 1)
        v = oracle.gemv_q4_mt(W[2], normed, kvd, H, nthr - 1)
        q = oracle.qkv_rope(q, k, v, ones_d, ones_d, kc, vc, nq, nkv, D, D, 0,
                            cfg["rope_theta_full"] if full else cfg["rope_theta"], eps,
                            ctx_len - 1, ctx_len - 1)
        a = oracle.decode_attn(q, kc, vc, slots_full if full else slots_sl, nq, D, kvd, nq // nkv)
        o = oracle.gemv_q4_mt(W[3], a, H, qd, nthr - 1)
        x, normed = oracle.add_rmsnorm(x, oracle.rmsnorm(o, ones_h, eps), ones_h, eps, 1.0)
        _, d = oracle.fused_mlp_step_mt(W[4], W[5], W[6], normed, H, I, nthr - 1)
        x, _ = oracle.add_rmsnorm(x, oracle.rmsnorm(d, ones_h, eps), ones_h, eps, 1.0)
        return x

    n, t0 = 0, time.perf_counter()
    while True:
        for li, W in layers:
            x = layer_step(li, W, x)
            n += 1
        if time.perf_counter() - t0 >= seconds:
            break
    t_layer = (time.perf_counter() - t0) / n
    rows = 16384
    E = oracle.synth_q8(rows, H, seed + 7, 0.0001, 0.0005)
    t1 = time.perf_counter()
    lg = oracle.gemv_q8_mt(E, x, rows, H, nthr - 1)
    t_logits = (time.perf_counter() - t1) * (cfg["vocab_size"] / rows)
    full_lg = np.resize(lg, cfg["vocab_size"])
    t2 = time.perf_counter()
    oracle.topk64(full_lg)
    t_topk = time.perf_counter() - t2
    t_tok = cfg["num_layers"] * t_layer + t_logits + t_topk
    return {"value": 1.0 / t_tok, "unit": "tok/s", "cores": nthr, "kind": "port",
            "sample": f"{n} decoder-layer steps (layers 0 and 4 of the 12B model, context {ctx_len}) "
                      f"at {t_layer * 1e3:.1f} ms each x 48, plus Q8 logits over 16384 of 262144 rows "
                      f"scaled ({t_logits * 1e3:.0f} ms) and one top-64 ({t_topk * 1e3:.0f} ms); "
                      f"{nthr} threads ({nthr - 1} pool workers + caller), {model}"}


def bench_decode(ctx, args):
    """Greedy decode through the recorded graph of the synthetic 12B model."""
    import numpy as np

    from channel_amd.model import Model

    cfg = CFG_12B
    H, I = cfg["hidden_size"], cfg["intermediate_size"]
    t_create = time.perf_counter()
    m = Model.synthetic(ctx, cfg, SEED)
    t_create = time.perf_counter() - t_create
    if args.eager:
        m.set_graph(False)
    rng = np.random.default_rng(SEED)
    prompt = rng.integers(0, cfg["vocab_size"], PROMPT).astype(np.uint32)
    slots = np.arange(PROMPT, dtype=np.uint32)
    # prefill twice: the first run warms code objects, the second is timed
    m.prefill_batch(prompt, slots, 0, 0, logits=False, topk=True)
    t0 = time.perf_counter()
    _, ids, _ = m.prefill_batch(prompt, slots, 0, 0, logits=False, topk=True)
    prefill_s = time.perf_counter() - t0

    # greedy decode on the device: the step parameters and the slot lists of
    # the 4096-slot ring are generated on the GPU, the argmax feeds the next
    # step's embedding gather; the timed region holds K decode tokens
    def greedy(tok, clock, n):
        out = []
        while n > 0:
            k = min(n, 4096)
            g = m.decode_greedy(tok, clock, k)
            out.append(g)
            tok, clock, n = int(g[-1]), clock + k, n - k
        return np.concatenate(out) if out else np.zeros(0, np.uint32)

    tok = int(ids[0])
    clock = PROMPT
    if args.warmup:
        tok = int(greedy(tok, clock, args.warmup)[-1])
        clock += args.warmup
    ctx.sync()
    ctx_start = clock
    t0 = time.perf_counter()
    ctx.timer_start()
    gen = greedy(tok, clock, args.steps)
    gpu_ms = ctx.timer_stop()
    wall_ms = (time.perf_counter() - t0) * 1e3
    clock += args.steps
    ms_per_tok = max(gpu_ms, wall_ms) / args.steps

    # the same steps driven token by token through the reference-shaped
    # interface (host slot lists uploaded per token, ids copied back)
    from channel_amd import ring
    window = cfg["sliding_window"]
    tok = int(gen[-1])
    n_api = 32
    t0 = time.perf_counter()
    for _ in range(n_api):
        slot, active, sliding = ring.decode_lists(clock, window)
        tok, _, _ = m.forward_token_id(tok, clock, slot, active, sliding)
        clock += 1
    api_ms = (time.perf_counter() - t0) * 1e3 / n_api
    mid_ctx = ctx_start + args.steps // 2
    w_bytes, kv_bytes = token_bytes(cfg, mid_ctx)
    m.close()

    # dominant kernel: fused gate/up matvec at the model's shape, rotating
    # distinct weight pairs, back to back on the library stream
    pairs = alloc_gateup_copies(ctx, H, I, repacked=True)
    x = ctx.alloc(H * 4)
    ctx.call("chn_synth_normal", x, H, SEED + 7, 1.0)
    act = ctx.alloc(I * 4)
    reps = max(192, 4 * len(pairs))
    k_ms = time_gateup(ctx, pairs, x, act, H, I, reps, repacked=True, fused_norm=True)
    achieved = gateup_bytes(H, I, fused_norm=True) / (k_ms * 1e-3) / 1e9
    read_gbps = gateup_bytes(H, I, repacked=True, fused_norm=True) / (k_ms * 1e-3) / 1e9
    sa_ms = time_gateup(ctx, pairs, x, act, H, I, reps, repacked=True)
    sa_gbps = gateup_bytes(H, I) / (sa_ms * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_decode_sample(cfg, SEED, mid_ctx, args.cpu_seconds)

    return {
        "value": 1e3 / ms_per_tok,
        "unit": "tok/s",
        "ms_per_step": ms_per_tok,
        "config": {"workload": "12B-class Q4 decode: 48 layers, hidden 3840, FFN 15360, 16 q / 8 kv heads, "
                               "head_dim 256, vocab 262144; 512-token prompt prefill, then greedy decode",
                   "prompt_tokens": PROMPT, "decode_context": [ctx_start, ctx_start + args.steps],
                   "decode_mode": "device-resident greedy steps (chn_decode_greedy)",
                   "api_tok_s": 1e3 / api_ms,
                   "prefill_tok_s": PROMPT / prefill_s, "prefill_ms": prefill_s * 1e3,
                   "token_weight_bytes": w_bytes, "token_kv_bytes_mid": kv_bytes,
                   "token_hbm_gbps": (w_bytes + kv_bytes) / (ms_per_tok * 1e-3) / 1e9,
                   "token_roofline_frac": (w_bytes + kv_bytes) / (ms_per_tok * 1e-3) / 1e9 / HBM_PEAK_GBS,
                   "model_create_s": t_create,
                   "decode_launch": "eager kernel launches" if args.eager else "HIP graph replay"},
        "roofline": {"kernel": "k_q4rmv_mlp_xp<8,NORM_POST_ADD> (chn_ffn_gate_up_q4r, the decode step's "
                               "launch: post-attention norm + residual + pre-FFN norm prologue, gate/up 15360x3840 "
                               "x2 + GELU-tanh * up + planes of act, repacked weights as the model holds them)",
                     "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": load_traffic("k_q4rmv_mlp_xp<8,2>", "gate/up 15360x3840"),
                     "algorithmic_bytes_per_launch": gateup_bytes(H, I, fused_norm=True),
                     "bytes_per_launch_repacked_layout": gateup_bytes(H, I, repacked=True, fused_norm=True),
                     # `achieved` counts the reference layout's 20 B per 32 weights (the
                     # algorithmic figure); the kernel streams the repacked 18 B layout,
                     # and this is its rate on the bytes it actually reads
                     "achieved_on_bytes_read": read_gbps, "frac_on_bytes_read": read_gbps / HBM_PEAK_GBS,
                     "avg_launch_ms": k_ms,
                     "standalone_from_planes": {
                         "kernel": "k_q4rmv_mlp_xp<4,-1> (chn_fused_mlp_q4r_xp: x's planes ready-made)",
                         "avg_launch_ms": sa_ms, "achieved": sa_gbps, "frac": sa_gbps / HBM_PEAK_GBS,
                         "algorithmic_bytes_per_launch": gateup_bytes(H, I),
                         "traffic": load_traffic("k_q4rmv_mlp_xp", "gate/up 15360x3840")}},
        "cpu_baseline": cpu,
        "dtype": DTYPE_DECODE,
        "data": "synthetic (seeded random-init 12B Q4 weights: codes uniform 0..15, f16 scales "
                "U(0.005, 0.02), norms 1, bf16 embedding ~ N(0, 0.02) tied to Q8 logits; prompt of "
                "uniform random token ids)",
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
    calls = [ctx.bind("chn_gemv_q4", w, x, y, M, K) for w in Ws]
    for i in range(args.warmup):
        calls[i % ncopy]()
    ctx.sync()
    t0 = time.perf_counter()
    ctx.timer_start()
    for i in range(args.steps):
        calls[i % ncopy]()
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
        "roofline": {"kernel": "k_q4mv<GEMV> (chn_gemv_q4: one launch, x's digit planes made in the kernel)", "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": load_traffic("k_q4mv<GEMV,XIN>", "8192x2048"),
                     "algorithmic_bytes_per_launch": nbytes, "avg_launch_ms": k_ms},
        "cpu_baseline": cpu,
        "dtype": DTYPE_Q4MV,
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
        "roofline": {"kernel": "k_q4gemm_p<1,128,REF> (128x128 tiles, DMA-pipelined K walk) + k_to_bf16 pre-pass",
                     "bound": "mfma",
                     "achieved": achieved, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / MFMA_BF16_PEAK_TFLOPS,
                     "traffic": load_traffic("k_q4gemm_p<1,128,REF>", "512x3840 -> 15360"),
                     "algorithmic_flop_per_launch": flops,
                     "avg_launch_ms": gpu_ms / args.steps},
        "cpu_baseline": None,
        "dtype": "bf16 MFMA operands, fp32 accumulate",
    }


def bench_attn(ctx, args):
    """Decode attention, 16 query / 8 KV heads, head_dim 256, over --slots
    entries (default the full 4096-slot ring) of fp32 K/V."""
    import numpy as np

    H, KVH, D, NSLOT = 16, 8, 256, 4096
    S = args.slots
    if not 1 <= S <= NSLOT:
        raise SystemExit(f"--slots must be in 1..{NSLOT}")
    kv_dim = KVH * D
    # caches of S rows, rotated over enough copies (> 512 MB) that no call
    # finds its K/V in the 256 MB Infinity Cache
    ncopy = max(4, -(-(512 << 20) // (2 * S * kv_dim * 4)))
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
    # a ring list of NSLOT entries whose slot values index the S cache rows
    slots = ctx.upload(((np.arange(NSLOT) + 1234) % S).astype(np.uint32))
    ns = ctx.upload(np.array([S], np.uint32))
    out = ctx.alloc(H * D * 4)
    ctx.sync()
    for i in range(args.warmup):
        ctx.call("chn_decode_attn", q, Kc[i % ncopy], Vc[i % ncopy], slots, ns, NSLOT, H, D, kv_dim, 2, 1.0, out)
    ctx.sync()
    t0 = time.perf_counter()
    ctx.timer_start()
    for i in range(args.steps):
        ctx.call("chn_decode_attn", q, Kc[i % ncopy], Vc[i % ncopy], slots, ns, NSLOT, H, D, kv_dim, 2, 1.0, out)
    gpu_ms = ctx.timer_stop()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms = max(gpu_ms, wall_ms) / args.steps
    nbytes = 2 * S * kv_dim * 4 + S * 4 + 2 * H * D * 4
    achieved = nbytes / (gpu_ms / args.steps * 1e-3) / 1e9
    # the same steps recorded once (one step per cache copy) and submitted
    # again, as the decode graph runs them
    ctx.record_begin()
    for i in range(ncopy):
        ctx.call("chn_decode_attn", q, Kc[i], Vc[i], slots, ns, NSLOT, H, D, kv_dim, 2, 1.0, out)
    rec = ctx.record_end()
    reps = max(1, -(-args.steps // ncopy))
    rec.submit()
    ctx.sync()
    ctx.timer_start()
    for _ in range(reps):
        rec.submit()
    rec_ms = ctx.timer_stop() / (reps * ncopy)
    rec.free()
    return {
        "value": 1e3 / ms, "unit": "attention steps/s", "ms_per_step": ms,
        "config": {"workload": f"decode attention over {S} of 4096 ring slots (16 q / 8 kv heads, D 256)",
                   "slots": S, "bytes_per_step": nbytes},
        "roofline": {"kernel": "k_attn_decode + k_attn_merge", "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": load_traffic("k_attn_decode + k_attn_merge", "4096 slots") if S == 4096 else None,
                     "algorithmic_bytes_per_launch": nbytes,
                     "avg_launch_ms": gpu_ms / args.steps,
                     "recorded": {"ms_per_step": rec_ms, "achieved": nbytes / (rec_ms * 1e-3) / 1e9,
                                  "frac": nbytes / (rec_ms * 1e-3) / 1e9 / HBM_PEAK_GBS}},
        "cpu_baseline": None,
        "dtype": "fp32",
    }


def bench_copy(ctx, args):
    """Device-to-device copy of 1 GiB (chn_copy): the HBM copy rate and the
    known-size kernel against which rocprofv3 FETCH_SIZE / WRITE_SIZE are
    calibrated."""
    n = 1 << 30
    src = ctx.alloc(n)
    dst = ctx.alloc(n)
    ctx.fill_u32(src, 0x3F800000, n // 4)
    ctx.sync()
    for _ in range(args.warmup):
        ctx.call("chn_copy", dst, src, n)
    ctx.sync()
    t0 = time.perf_counter()
    ctx.timer_start()
    for _ in range(args.steps):
        ctx.call("chn_copy", dst, src, n)
    gpu_ms = ctx.timer_stop()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms = max(gpu_ms, wall_ms) / args.steps
    achieved = 2 * n / (gpu_ms / args.steps * 1e-3) / 1e9
    return {
        "value": 2 * n / (ms * 1e-3) / 1e9, "unit": "GB/s (read + write)", "ms_per_step": ms,
        "config": {"workload": "device copy of 1 GiB (chn_copy)", "bytes_copied": n},
        "roofline": {"kernel": "device copy", "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "algorithmic_bytes_per_launch": 2 * n, "avg_launch_ms": gpu_ms / args.steps},
        "cpu_baseline": None,
        "dtype": "bytes",
        "data": "constant fill",
    }


WORKLOADS = {"decode": bench_decode, "mlp": bench_mlp, "gemv": bench_gemv, "prefill": bench_prefill,
             "attn": bench_attn, "copy": bench_copy}
DEFAULT_STEPS = {"decode": (256, 8), "copy": (20, 2)}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="decode", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--slots", type=int, default=4096, help="attn workload: slot count (<= 4096)")
    ap.add_argument("--layout", default="q4r", choices=["q4r", "q4"],
                    help="mlp workload: repacked weights as the model holds them, or the reference layout")
    ap.add_argument("--eager", action="store_true",
                    help="decode: launch the kernels one by one instead of replaying the graph")
    args = ap.parse_args()
    d_steps, d_warm = DEFAULT_STEPS.get(args.workload, (200, 20))
    args.steps = d_steps if args.steps is None else args.steps
    args.warmup = d_warm if args.warmup is None else args.warmup
    if args.steps < 1 or args.warmup < 0:
        ap.error("--steps must be >= 1 and --warmup >= 0")

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures the single-GPU hot path only; run it with --gpus 1 "
              "(there is no multi-GPU path to measure).", file=sys.stderr)
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
        "data": r.get("data", "synthetic (seeded; Q4 codes uniform 0..15, f16 scales U(0.005, 0.02), "
                              "x ~ N(0,1))"),
        "config": r["config"],
        "roofline": r["roofline"],
        "cpu_baseline": r["cpu_baseline"],
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
