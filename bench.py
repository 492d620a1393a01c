"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline (the `value`): configs[1] of BASELINE.json at M=1, 4-bit g64 -- decode over
32 distinct Llama-3-8B MLP layers (gate, up [14336,4096] and down [4096,14336]),
one step = the 96 qmv launches of one token. value = algorithmic HBM bytes moved
per second (TB/s), weights resident in HBM, synthetic data from the library's
generator. The JSON line also carries the roofline of the dominant kernel, the
timed CPU baseline (the C oracle, not MLX) and the secondary configs.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--full]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mlx-serve_amd"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
SEED_BASE = 0x4D49333500000000


def seed(cfg, stream, extra=0):
    return (SEED_BASE + 16 * cfg + stream + (extra << 20)) & ((1 << 64) - 1)


FP_MODES = {"nvfp4": (16, 4), "mxfp4": (32, 4), "mxfp8": (32, 8)}  # (group_size, bits)


def qbytes(N, K, bits, gs, M, mode="affine"):
    """Algorithmic bytes of one qmm call: packed W + scales (+ biases) + x + y. Affine
    scales/biases are bf16; the fp modes have one uint8 scale per group and no biases."""
    sb = N * K // gs if mode in FP_MODES else 2 * (N * K // gs) * 2
    return N * K * bits // 8 + sb + M * K * 2 + M * N * 2


def build_fp_layers(torch, n_layers, mode, dev, hidden=4096, inter=14336):
    """Random codes and scales for a bias-less fp mode (near-unit scales; every code)."""
    gs, bits = FP_MODES[mode]
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed(2, 1))
    lo, hi = (0x20, 0x48) if mode == "nvfp4" else (118, 126)

    def one(N, K):
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K * bits // 32), generator=gen,
                          device=dev, dtype=torch.int32)
        sc = torch.randint(lo, hi, (N, K // gs), generator=gen, device=dev, dtype=torch.uint8)
        return (w, sc, None)

    layers = [(one(inter, hidden), one(inter, hidden), one(hidden, inter))
              for _ in range(n_layers)]
    torch.cuda.synchronize()
    return layers


def make_layer_weights(torch, mi, N, K, bits, gs, sd, tmp):
    w = tmp[: N * K].view(N, K)
    mi.fill_randn(w, sd, 0.0, 0.02)
    return mi.quantize(w, gs, bits)


def build_mlp_layers(torch, mi, n_layers, bits, gs, dev, hidden=4096, inter=14336, cfg=2):
    tmp = torch.empty(hidden * inter, dtype=torch.bfloat16, device=dev)
    layers = []
    for l in range(n_layers):
        g = make_layer_weights(torch, mi, inter, hidden, bits, gs, seed(cfg, 1, 3 * l), tmp)
        u = make_layer_weights(torch, mi, inter, hidden, bits, gs, seed(cfg, 1, 3 * l + 1), tmp)
        d = make_layer_weights(torch, mi, hidden, inter, bits, gs, seed(cfg, 1, 3 * l + 2), tmp)
        layers.append((g, u, d))
    del tmp
    torch.cuda.synchronize()
    return layers


def time_region(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / 1000.0


def decode_mlp(torch, mi, layers, M, bits, gs, dev, steps, warmup, hidden=4096, inter=14336,
               mode="affine"):
    x = torch.empty(M, hidden, dtype=torch.bfloat16, device=dev)
    h = torch.empty(M, inter, dtype=torch.bfloat16, device=dev)
    mi.fill_randn(x, seed(2, 0), 0.0, 1.0)
    mi.fill_randn(h, seed(2, 0, 1), 0.0, 1.0)

    def step():
        for (g, u, d) in layers:
            mi.quantized_matmul(x, *g, True, gs, bits, mode)
            mi.quantized_matmul(x, *u, True, gs, bits, mode)
            mi.quantized_matmul(h, *d, True, gs, bits, mode)

    # The 96 launches of one token are captured once in a HIP graph and replayed, so
    # the timed region measures the GPU, not Python's per-call launch overhead.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    t = time_region(torch, graph.replay, steps, warmup)
    launches = 3 * len(layers) * steps
    per_launch = qbytes(inter, hidden, bits, gs, M, mode)  # gate/up/down move the same bytes
    return {"seconds": t, "launches": launches, "bytes_per_launch": per_launch,
            "avg_launch_us": t / launches * 1e6,
            "GBs": per_launch * launches / t / 1e9,
            "tokens_per_s": M * steps / t}


def single_qmv(torch, mi, dev, reps=50, warmup=5):
    """one 4-bit g64 qmv x [1,4096] @ W [4096,4096]^T. Reports the eager
    single-call latency (HIP events bracketing one Python/ctypes call on an idle GPU, median:
    it includes the host-side enqueue, so it is a host-inclusive latency, not a kernel time)
    and the rate over rotated copies (>= 512 MB in one graph, so each call streams its weight
    from HBM; that is the kernel figure)."""
    N = K = 4096
    bits, gs = 4, 64
    per = qbytes(N, K, bits, gs, 1)
    copies = -(-512 * 10 ** 6 // per)
    tmp = torch.empty(N, K, dtype=torch.bfloat16, device=dev)
    Ws = []
    for c in range(copies):
        mi.fill_randn(tmp, seed(1, 1, c), 0.0, 0.02)
        Ws.append(mi.quantize(tmp, gs, bits))
    del tmp
    x = torch.empty(1, K, dtype=torch.bfloat16, device=dev)
    mi.fill_randn(x, seed(1, 0), 0.0, 1.0)
    for _ in range(warmup):
        mi.quantized_matmul(x, *Ws[0], True, gs, bits)
    torch.cuda.synchronize()
    lat = []
    for r in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        mi.quantized_matmul(x, *Ws[r % copies], True, gs, bits)
        b.record()
        torch.cuda.synchronize()
        lat.append(a.elapsed_time(b) * 1e3)
    lat.sort()

    def all_copies():
        for W in Ws:
            mi.quantized_matmul(x, *W, True, gs, bits)
    t = graph_time(torch, all_copies, 10, 2) / copies
    return {"cfg0_single_call_host_inclusive_latency_us": round(lat[len(lat) // 2], 2),
            "cfg0_rotated_us_per_call": round(t * 1e6, 3),
            "cfg0_rotated_GBs": round(per / t / 1e9, 1),
            "cfg0_rotated_copies": copies}


def cpu_info():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return model, os.cpu_count() or 1, avail


def check_sample(torch, layers, x, y_fn, bits, gs, hidden=4096):
    """Bench-time correctness gate: the first layer's gate output for the benchmark's own
    x against the C oracle (fp64), before any number is reported."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as O
    g = layers[0][0]
    y = y_fn(x, g)
    wq = g[0].cpu().numpy().view(np.uint32)
    s = g[1].cpu().view(torch.int16).numpy().view(np.uint16)
    b = g[2].cpu().view(torch.int16).numpy().view(np.uint16)
    xh = x.cpu().view(torch.int16).numpy().view(np.uint16)
    truth = O.qmm_f64(xh, wq, s, b, gs, bits)
    err = float(np.max(np.abs(y.float().cpu().numpy() - truth)) / np.max(np.abs(truth)))
    if not err <= 1e-2:
        raise SystemExit(f"bench correctness gate failed: rel-err {err:.3e}")
    return err


def cpu_baseline(torch, layers, bits, gs, hidden=4096, inter=14336, budget_s=10.0):
    """Time the C oracle's fp32 qmv (a C restatement of MLX CPU semantics, not MLX)
    on host cores over a bounded sample: the first layers' weights copied to host."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as O
    model, ncpu, avail = cpu_info()
    threads = min(16, avail)  # the GPU box's CPU share is 16 threads
    n_l = min(4, len(layers))
    host = []
    for (g, u, d) in layers[:n_l]:
        host.append([tuple(t.cpu().view(torch.int16 if t.element_size() == 2 else torch.int32)
                           .numpy() for t in m) for m in (g, u, d)])
    host = [[(wq.view(np.uint32), s.view(np.uint16), b.view(np.uint16)) for (wq, s, b) in L]
            for L in host]
    x = O.make_x_bf16(1, hidden, seed(2, 0))
    h = O.make_x_bf16(1, inter, seed(2, 0, 1))
    O.qmm_f32(x, *host[0][0], gs, bits, threads)  # warm
    done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        for L in host:
            O.qmm_f32(x, *L[0], gs, bits, threads)
            O.qmm_f32(x, *L[1], gs, bits, threads)
            O.qmm_f32(h, *L[2], gs, bits, threads)
            done += 3
    t = time.perf_counter() - t0
    per = qbytes(inter, hidden, bits, gs, 1)
    return {"value": per * done / t / 1e12, "unit": "TB/s", "cores": threads, "kind": "port",
            "cpu_model": model, "nproc": ncpu, "affinity_cpus": avail, "threads": threads,
            "sample": f"{done} qmv calls (M=1, 4-bit g64, Llama-3-8B MLP shapes) over the first "
                      f"{n_l} layers' weights, {t:.1f} s, C oracle mo_qmm_f32 (fp32, C "
                      f"restatement of MLX CPU semantics, not MLX) with {threads} OpenMP threads"}


def graph_time(torch, fn, replays, warmup=2):
    """Capture fn() once in a HIP graph (after an eager warm-up that sizes the library
    workspace) and return seconds per replay."""
    fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    return time_region(torch, graph.replay, replays, warmup) / replays


def prefill(torch, mi, dev, Ms, steps=10, warmup=2, bits=4, gs=64):
    """prefill qmm TFLOP/s for x [M, K] against 4-bit g64 W [N, K] (other widths
    with --bits: 8-bit on the fused prefill kernel, 2/3/5/6 through dequantize + the bf16
    GEMM)."""
    out = {}
    for (N, K, name) in ((14336, 4096, "gate"), (4096, 14336, "down")):
        tmp = torch.empty(N * K, dtype=torch.bfloat16, device=dev).view(N, K)
        mi.fill_randn(tmp, seed(3, 1), 0.0, 0.02)
        W = mi.quantize(tmp, gs, bits)
        del tmp
        for M in Ms:
            x = torch.empty(M, K, dtype=torch.bfloat16, device=dev)
            mi.fill_randn(x, seed(3, 0, M), 0.0, 1.0)
            t = time_region(torch, lambda: mi.quantized_matmul(x, *W, True, gs, bits), steps,
                            warmup)
            tf = 2.0 * M * N * K * steps / t / 1e12
            tag = f"prefill_{name}_M{M}" if bits == 4 else f"prefill{bits}_{name}_M{M}"
            out[f"{tag}_TFLOPs"] = round(tf, 1)
            out[f"{tag}_pct_bf16_peak"] = round(100 * tf / BF16_PEAK_TFLOPS, 2)
            out[f"{tag}_tok_s"] = round(M * steps / t, 1)
        del W
    return out


def moe_bank(torch, mi, dev, E, N, K, bits, gs, sd):
    tmp = torch.empty(E * N * K, dtype=torch.bfloat16, device=dev).view(E * N, K)
    mi.fill_randn(tmp, sd, 0.0, 0.02)
    wq, s, b = mi.quantize(tmp, gs, bits)
    return wq.view(E, N, -1), s.view(E, N, -1), b.view(E, N, -1)


def moe_layer(torch, mi, dev, cfg, E, hidden, inter, k, Ts, n_routes=16, steps=10, warmup=2,
              skew=False):
    """configs[3]/[4]: one routed-expert MoE layer (route -> gate/up -> SwiGLU -> down ->
    score-weighted sum), 4-bit g64, decode (T=1, fused entry points) and sorted prefill.
    Routings differ per iteration so the touched experts are not cache-resident.
    GB/s counts each distinct expert's packed + scale/bias bytes once, plus activations."""
    bits, gs = 4, 64
    G = moe_bank(torch, mi, dev, E, inter, hidden, bits, gs, seed(cfg, 1, 1))
    U = moe_bank(torch, mi, dev, E, inter, hidden, bits, gs, seed(cfg, 1, 2))
    D = moe_bank(torch, mi, dev, E, hidden, inter, bits, gs, seed(cfg, 1, 3))
    per_expert = 3 * (inter * hidden * bits // 8 + 2 * (inter * hidden // gs) * 2)
    out = {}
    for T in Ts:
        logits = torch.empty(n_routes, T, E, dtype=torch.float32, device=dev)
        mi.fill_randn(logits, seed(cfg, 2, T), 0.0, 1.0)
        if skew:
            # 10% of tokens pushed onto 8 fixed hot experts (+8.0 on their logits)
            g = torch.Generator().manual_seed(seed(cfg, 3) & 0x7FFFFFFF)
            hot = torch.randperm(E, generator=g)[:8]
            pick = torch.rand(n_routes, T, generator=g) < 0.1
            bump = torch.zeros(n_routes, T, E)
            bump[:, :, hot] = 8.0
            logits += (bump * pick[..., None]).to(dev)
        x = torch.empty(T, hidden, dtype=torch.bfloat16, device=dev)
        mi.fill_randn(x, seed(cfg, 0, T), 0.0, 1.0)
        routes = [mi.moe_route_topk(logits[r], k, torch.bfloat16) for r in range(n_routes)]
        distinct = [torch.unique(r[0]).numel() for r in routes]

        def layer(r):
            if T == 1:
                # routing runs inside the gate + up launch (2 launches per layer)
                act, inds, sc = mi.moe_route_gate_up_swiglu(logits[r], x, *G, *U, k, gs, bits)
                return mi.gather_qmv_down_reduce(act, *D, inds, sc, gs, bits)
            inds, sc = mi.moe_route_topk(logits[r], k, torch.bfloat16)
            order, inv, srt, lhs, seg = mi.moe_sort_dispatch(inds.reshape(-1), k, E)
            xs = x.view(T, 1, hidden)
            # gate and up in one call with SwiGLU applied as it writes; the un-sort rides in
            # the slot reduce
            a = mi.gather_qmm_gate_up_swiglu(xs, *G, *U, lhs_indices=lhs, rhs_indices=srt,
                                             group_size=gs, bits=bits, sorted_indices=True)
            v = mi.gather_qmm(a, *D, rhs_indices=srt, group_size=gs, bits=bits,
                              sorted_indices=True)
            return mi.moe_down_reduce_rows(v.view(T * k, hidden), inv, sc)

        def all_routes():
            for r in range(n_routes):
                layer(r)

        # one graph = n_routes layer steps, each with its own routing
        t = graph_time(torch, all_routes, steps, warmup) / n_routes
        avg_distinct = sum(distinct) / len(distinct)
        byts = avg_distinct * per_expert + T * hidden * 2 * 2 + T * k * inter * 2 * 3
        out[f"moe{cfg + 1}_T{T}_us"] = round(t * 1e6, 1)
        out[f"moe{cfg + 1}_T{T}_GBs"] = round(byts / t / 1e9, 1)
        out[f"moe{cfg + 1}_T{T}_tok_s"] = round(T / t, 1)
        out[f"moe{cfg + 1}_T{T}_distinct_experts"] = round(avg_distinct, 1)
    return out


def shared_expert_8bit(torch, mi, dev, Ts, steps=10, warmup=2):
    """configs[4] shared expert: 8-bit g64 dense MLP (2048,7168)x2 + (7168,2048)."""
    bits, gs = 8, 64
    mats = []
    for (N, K, st) in ((2048, 7168, 4), (2048, 7168, 5), (7168, 2048, 6)):
        tmp = torch.empty(N * K, dtype=torch.bfloat16, device=dev).view(N, K)
        mi.fill_randn(tmp, seed(4, 1, st), 0.0, 0.02)
        mats.append(mi.quantize(tmp, gs, bits))
    out = {}
    for T in Ts:
        x = torch.empty(T, 7168, dtype=torch.bfloat16, device=dev)
        h = torch.empty(T, 2048, dtype=torch.bfloat16, device=dev)
        mi.fill_randn(x, seed(4, 0, T), 0.0, 1.0)
        mi.fill_randn(h, seed(4, 0, T + 1), 0.0, 1.0)

        def step():
            mi.quantized_matmul(x, *mats[0], True, gs, bits)
            mi.quantized_matmul(x, *mats[1], True, gs, bits)
            mi.quantized_matmul(h, *mats[2], True, gs, bits)

        t = graph_time(torch, step, steps * 5, warmup)
        byts = sum(qbytes(N, K, bits, gs, T) for (N, K) in ((2048, 7168), (2048, 7168),
                                                           (7168, 2048)))
        out[f"shared8_T{T}_GBs"] = round(byts / t / 1e9, 1)
        out[f"shared8_T{T}_us"] = round(t * 1e6, 1)
    return out


def pmc_traffic():
    """HBM bytes per decode launch, from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (counters scaled by a copy kernel of known size); None if absent."""
    path = os.path.join(ROOT, "profiles", "qmv1_decode_llama8b_mlp_pmc_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--decode-only", type=int, default=0, metavar="M",
                    help="only run the configs[1] decode step at this M (for rocprofv3)")
    ap.add_argument("--bits", type=int, default=4, choices=(2, 3, 4, 5, 6, 8),
                    help="weight bits of --decode-only and --prefill-only")
    ap.add_argument("--mode", default="affine", choices=("affine",) + tuple(FP_MODES),
                    help="weight format of --decode-only (fp modes: random codes and scales)")
    ap.add_argument("--prefill-only", type=int, default=0, metavar="M",
                    help="only run the configs[2] prefill shapes at this M (for rocprofv3)")
    ap.add_argument("--moe-only", type=int, default=0, choices=(0, 3, 4), metavar="CFG",
                    help="only run the MoE layer of configs[CFG] (3 or 4; for rocprofv3)")
    ap.add_argument("--tokens", type=int, default=0, help="T of --moe-only (default: all)")
    ap.add_argument("--shared-only", type=int, default=0, metavar="T",
                    help="time only configs[4]'s 8-bit shared expert at T tokens")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 4 device copies of 256 MiB (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE/WRITE_SIZE to bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build's path runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured configuration).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        a = torch.empty(1 << 27, dtype=torch.int16, device=dev)
        b = torch.empty_like(a)
        for _ in range(4):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_each_way": a.numel() * 2, "copies": 4}))
        return
    import mi_qmm as mi
    if args.decode_only:
        if args.mode in FP_MODES:
            gs, bits = FP_MODES[args.mode]
            layers = build_fp_layers(torch, args.layers, args.mode, dev)
        else:
            gs, bits = 64, args.bits
            layers = build_mlp_layers(torch, mi, args.layers, bits, gs, dev)
        r = decode_mlp(torch, mi, layers, args.decode_only, bits, gs, dev, args.steps,
                       args.warmup, mode=args.mode)
        print(json.dumps({"M": args.decode_only, "bits": bits, "mode": args.mode,
                          "GBs": round(r["GBs"], 1), "avg_launch_us": round(r["avg_launch_us"], 3),
                          "bytes_per_launch": r["bytes_per_launch"]}))
        return
    if args.prefill_only:
        print(json.dumps(prefill(torch, mi, dev, (args.prefill_only,), steps=args.steps,
                                 warmup=args.warmup, bits=args.bits)))
        return
    if args.shared_only:
        print(json.dumps(shared_expert_8bit(torch, mi, dev, (args.shared_only,))))
        return
    if args.moe_only:
        if args.moe_only == 3:
            Ts = (args.tokens,) if args.tokens else (1, 512)
            r = moe_layer(torch, mi, dev, 3, 128, 2048, 768, 8, Ts)
        else:
            Ts = (args.tokens,) if args.tokens else (1, 8, 64)
            r = moe_layer(torch, mi, dev, 4, 256, 7168, 2048, 8, Ts, skew=True)
            r.update(shared_expert_8bit(torch, mi, dev, Ts))
        print(json.dumps(r))
        return
    bits, gs = 4, 64
    layers = build_mlp_layers(torch, mi, args.layers, bits, gs, dev)
    head = decode_mlp(torch, mi, layers, 1, bits, gs, dev, args.steps, args.warmup)
    xg = torch.empty(1, 4096, dtype=torch.bfloat16, device=dev)
    mi.fill_randn(xg, seed(2, 0), 0.0, 1.0)
    gate_err = check_sample(torch, layers, xg,
                            lambda x, g: mi.quantized_matmul(x, *g, True, gs, bits), bits, gs)

    extra = {}
    if not args.no_extra:
        for M in (2, 4, 8, 16, 32):
            r = decode_mlp(torch, mi, layers, M, bits, gs, dev, max(5, args.steps // 5), 2)
            extra[f"q4_M{M}_GBs"] = round(r["GBs"], 1)
            extra[f"q4_M{M}_tok_s"] = round(r["tokens_per_s"], 1)
        del layers
        torch.cuda.empty_cache()
        layers8 = build_mlp_layers(torch, mi, args.layers, 8, gs, dev)
        for M in (1, 8, 32):
            r = decode_mlp(torch, mi, layers8, M, 8, gs, dev, max(5, args.steps // 5), 2)
            extra[f"q8_M{M}_GBs"] = round(r["GBs"], 1)
            extra[f"q8_M{M}_tok_s"] = round(r["tokens_per_s"], 1)
        del layers8
        torch.cuda.empty_cache()
        # the other formats at M = 1 and 8 (16 layers: 0.5 GB and up, beyond the caches)
        for b in (2, 3, 5, 6):
            lo = build_mlp_layers(torch, mi, 16, b, gs, dev)
            for M in (1, 8):
                r = decode_mlp(torch, mi, lo, M, b, gs, dev, max(5, args.steps // 5), 2)
                extra[f"q{b}_M{M}_GBs"] = round(r["GBs"], 1)
            del lo
            torch.cuda.empty_cache()
        for fm, (fgs, fb) in FP_MODES.items():
            lo = build_fp_layers(torch, 16, fm, dev)
            for M in (1, 8):
                r = decode_mlp(torch, mi, lo, M, fb, fgs, dev, max(5, args.steps // 5), 2,
                               mode=fm)
                extra[f"{fm}_M{M}_GBs"] = round(r["GBs"], 1)
            del lo
            torch.cuda.empty_cache()
        extra.update(single_qmv(torch, mi, dev))
        extra.update(prefill(torch, mi, dev, (512, 2048, 8192)))
        extra.update(moe_layer(torch, mi, dev, 3, 128, 2048, 768, 8, (1, 512)))
        extra.update(moe_layer(torch, mi, dev, 4, 256, 7168, 2048, 8, (1, 8, 64), skew=True))
        extra.update(shared_expert_8bit(torch, mi, dev, (1, 8, 64)))
        layers = None

    cpu = None
    if not args.no_cpu:
        if layers is None:
            layers = build_mlp_layers(torch, mi, 4, bits, gs, dev)
        cpu = cpu_baseline(torch, layers, bits, gs, budget_s=args.cpu_seconds)

    ms_per_step = head["seconds"] / args.steps * 1e3
    achieved = head["bytes_per_launch"] / (head["avg_launch_us"] * 1e-6) / 1e9
    out = {
        "metric": "4-bit qmv/gather_qmm HBM TB/s (% of peak) at M=1; prefill qmm TFLOP/s",
        "value": round(head["GBs"] / 1000.0, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 weights, bf16 activations, fp32 accumulate",
        "data": "synthetic (counter-based SplitMix64 normal, quantized on device)",
        "config": {"workload": "configs[1]: Llama-3-8B MLP decode, 32 distinct layers "
                               "(gate/up [14336,4096], down [4096,14336]), 4-bit g64, M=1",
                   "global_batch": 1, "layers": args.layers, "pct_of_hbm_peak":
                   round(100.0 * head["GBs"] / HBM_PEAK_GBS, 2),
                   "tokens_per_s": round(head["tokens_per_s"], 1),
                   "gate_rel_err_vs_oracle": float(f"{gate_err:.3e}")},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": pmc_traffic(), "kernel": "mi::qmv1_kernel<64, NC, DEPTH, true> (dense M=1 instances)",
                     "bytes_per_launch": head["bytes_per_launch"],
                     "avg_launch_us": round(head["avg_launch_us"], 3)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
