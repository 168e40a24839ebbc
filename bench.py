"""Benchmark of the GGUF quantized-linear decode path on one MI355X.

Workload (benchmark config 2, "the metric's configuration"): one Llama-3-8B-shaped layer's decode projections
at M = 1 with the Q4_K_M mix — q 4096x4096, k/v 1024x4096, o 4096x4096, gate/up 14336x4096 in Q4_K, down
4096x14336 in Q6_K. Weights N(0, 0.02) from a seed, quantised on the device with the reference quantizer
(GgmlQuant.QuantizeQ4_K) and the library's Q6_K encoder; activations N(0, 1) fp32, resident in HBM.

One step = the layer's four distinct activations quantised to Q8_K and its seven projections, in four launches
(each launch quantises its fp32 activation in-kernel, then runs its projections): fused q/k/v, o, fused
gate/up, down.
To measure HBM rather than the 256 MB Infinity Cache, steps rotate over several independent layer copies
(> 2x the cache). value = algorithmic bytes per step / time per step (weights + fp32 activations read once
+ fp32 outputs), in GB/s; decode_proj_tok_s = steps per second.

Also reported: the dominant kernel's roofline (the fused gate/up Q4_K GEMV, per-launch HIP-event timing on
the stream it runs on), benchmark config 1 (a single Q4_K 4096x4096 GEMV rotated over 64 copies), config 3
(the layer at M = 512 on int8 MFMA, with its MFMA roofline), config 4 (32 distinct layers + the Q6_K LM head,
one token's projections), config 5 (a Mixtral-shaped routed MoE step of 16 tokens), and the CPU baseline (the AVX2 C restatement of the reference's CPU path, on a
bounded sample, rank 0 only).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K GEMV HBM GB/s (% peak) + decode proj tok/s, Llama-3-8B shape"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
LAYER = [  # name, out, in, format
    ("q", 4096, 4096, "q4k"), ("k", 1024, 4096, "q4k"), ("v", 1024, 4096, "q4k"), ("o", 4096, 4096, "q4k"),
    ("gate", 14336, 4096, "q4k"), ("up", 14336, 4096, "q4k"), ("down", 4096, 14336, "q6k"),
]
BPB = {"q4k": 144, "q6k": 210}


def weight_bytes(n, k, fmt):
    return n * (k // 256) * BPB[fmt]


def layer_algorithmic_bytes():
    w = sum(weight_bytes(n, k, f) for _, n, k, f in LAYER)
    x = 4 * (4096 + 4096 + 4096 + 14336)          # distinct fp32 inputs: attn-in, o-in, ffn-in, down-in
    y = 4 * sum(n for _, n, _, _ in LAYER)        # fp32 outputs
    return w, w + x + y


def make_layer(ov, torch, seed):
    gen = torch.Generator(device="cuda:0").manual_seed(seed)
    ws = {}
    for name, n, k, fmt in LAYER:
        wf = torch.randn(n, k, generator=gen, device="cuda:0") * 0.02
        blocks = ov.quantize_weight(wf, ov.TYPE_Q6_K if fmt == "q6k" else ov.TYPE_Q4_K)
        del wf
        ws[name] = (ov.Q6KWeight if fmt == "q6k" else ov.Q4KWeight)(blocks, k, n)
        ws[name + "_blocks"] = blocks
    return ws


def cpu_meta(L, workers):
    """What the CPU baseline ran on and with: model, logical CPUs, the CPUs this process may use, worker threads,
    compiler and flags of the AVX2 restatement."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count() or 1
    info = L.cpub_build_info().decode()
    compiler, _, flags = info.partition("; ")
    return {"cpu_model": model, "nproc": os.cpu_count(), "cpus_allowed": allowed, "workers": workers,
            "compiler": compiler, "flags": flags}


def batched_workers():
    """OverfitParallel.For uses every core (WorkerCount = ProcessorCount); here the CPUs this process may use,
    capped at the 16 host CPUs one GPU's share of the box has."""
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count() or 1
    return max(1, min(allowed, 16))


def best_of(fn, budget_s, min_reps=3):
    fn()
    best, n = float("inf"), 0
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or n < min_reps:
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
        n += 1
    return best, n


def run_cpu_baseline(layer0_host, budget_s=2.5):
    """Times the AVX2 C restatement of the reference's decode path on one layer step (7 projections)."""
    import numpy as np

    import oracle

    L = oracle.lib()
    if not L.cpub_has_avx2():
        return None
    allowed = batched_workers()
    workers = max(1, min(allowed, 10))  # OverfitParallel decode cap min(cores, 10)
    L.cpub_set_workers(allowed)
    L.cpub_set_decode_cap(workers)
    rng = np.random.default_rng(1)
    xs = {k: rng.standard_normal(k).astype(np.float32) for k in (4096, 14336)}
    q = np.zeros(14336, np.int8)
    s = np.zeros(14336 // 256, np.float32)
    b = np.zeros(14336 // 16, np.int16)
    out = {name: np.zeros(n, np.float32) for name, n, _, _ in LAYER}
    P = oracle.P

    def step():
        x = xs[4096]
        L.cpub_quantize_q8k(P(x), 4096, P(q), P(s), P(b))   # shared attention input (quantised once)
        for name in ("q", "k", "v"):
            L.cpub_q4k_project_prequantized_parallel(P(layer0_host[name]), 4096, out[name].size, None,
                                                     P(out[name]), P(q), P(s), P(b))
        L.cpub_q4k_project_parallel(P(x), P(layer0_host["o"]), 4096, 4096, None, P(out["o"]), P(q), P(s), P(b))
        L.cpub_q4k_project_gate_up(P(x), P(layer0_host["gate"]), P(layer0_host["up"]), 4096, 14336,
                                   P(out["gate"]), P(out["up"]), P(q), P(s), P(b))
        L.cpub_q6k_project_parallel(P(xs[14336]), P(layer0_host["down"]), 14336, 4096, None, P(out["down"]),
                                    P(q), P(s), P(b))

    best, n = best_of(step, budget_s)
    _, alg = layer_algorithmic_bytes()
    line = {
        "value": round(alg / best / 1e9, 2),
        "unit": "GB/s",
        "tok_s": round(1.0 / best, 2),
        "ms_per_step": round(best * 1e3, 3),
        "cores": workers,
        "kind": "port",
        "sample": f"best of {n} steps of the config-2 layer (7 projections, same Q4_K/Q6_K bytes as the GPU run), "
                  f"AVX2 C restatement of Overfit's CPU path, {workers} row-band workers (ForDecode), "
                  f"~{budget_s:.1f}s wall",
    }
    line.update(cpu_meta(L, workers))
    return line


def run_cpu_configs(layer0_host, moe_host, budget_s=2.0):
    """CPU baselines of the other benchmark configurations, on the same bytes as the GPU run: config 1 (a Q4_K
    4096x4096 GEMV, ForDecode over min(cores, 10) bands), config 3 (the layer's seven projections at M = 512 through
    BatchedQuantProjection.Dispatch: Q4_K weight-stationary 64-row tiles, Q6_K ProjectBatched, OverfitParallel.For over
    every worker) and config 5 (MoeFeedForwardBlock.DecodeBatched over the routed tokens: per expert, the batched
    SwiGLU through the same Dispatch). Bit-identical to the oracle (tests/test_oracle_pins.py)."""
    import ctypes

    import numpy as np

    import oracle

    L = oracle.lib()
    if not L.cpub_has_avx2():
        return None
    P = oracle.P
    allw = batched_workers()
    dec = max(1, min(allw, 10))
    L.cpub_set_workers(allw)
    L.cpub_set_decode_cap(dec)
    rng = np.random.default_rng(3)
    out = {}

    # config 1: Q4_K 4096x4096 GEMV (the layer's q weight has exactly this shape)
    x1 = rng.standard_normal(4096).astype(np.float32)
    y1 = np.zeros(4096, np.float32)
    q = np.zeros(512 * 14336, np.int8)
    s = np.zeros(512 * 14336 // 256, np.float32)
    b = np.zeros(512 * 14336 // 16, np.int16)
    best, n = best_of(lambda: L.cpub_q4k_project_parallel(P(x1), P(layer0_host["q"]), 4096, 4096, None, P(y1),
                                                          P(q), P(s), P(b)), budget_s / 2)
    nbytes = weight_bytes(4096, 4096, "q4k") + 4 * 4096 + 4 * 4096
    out["config1_q4k_gemv_4096x4096"] = dict(
        value=round(nbytes / best / 1e9, 2), unit="GB/s", us=round(best * 1e6, 1), cores=dec, kind="port",
        sample=f"best of {n} Q4KDotKernel.ProjectParallel calls (quantise + {dec} row bands)", **cpu_meta(L, dec))

    # config 3: the layer at M = 512, seven Dispatch calls (each quantises its input rows, as the reference does)
    m = 512
    xin = {kk: rng.standard_normal(m * kk).astype(np.float32) for kk in (4096, 14336)}
    ys = {name: np.zeros(m * nn, np.float32) for name, nn, _, _ in LAYER}

    def prefill():
        for name, nn, kk, fmt in LAYER:
            fn = L.cpub_q6k_project_batched if fmt == "q6k" else L.cpub_q4k_project_batched_ws
            fn(P(xin[kk]), m, P(layer0_host[name]), kk, nn, None, P(ys[name]), P(q), P(s), P(b))

    best, n = best_of(prefill, budget_s, min_reps=2)
    ops = 2 * m * sum(nn * kk for _, nn, kk, _ in LAYER)
    out["config3_prefill_m512"] = dict(
        value=round(m / best, 1), unit="tokens/s", us_per_layer=round(best * 1e6, 1),
        useful_TOPS=round(ops / best / 1e12, 3), cores=allw, kind="port",
        sample=f"best of {n} layer steps at M={m} (7 BatchedQuantProjection.Dispatch calls: Q4_K weight-stationary, "
               f"Q6_K batched; OverfitParallel.For over {allw} workers)", **cpu_meta(L, allw))

    # config 5: the routed MoE step on the GPU run's expert bytes, routing and tokens
    if moe_host is not None:
        E = len(moe_host["gate"])
        arr = lambda ms: (ctypes.c_void_p * E)(*[mm.ctypes.data for mm in ms])  # noqa: E731
        G, U, D = arr(moe_host["gate"]), arr(moe_host["up"]), arr(moe_host["down"])
        xm, idx, wts = moe_host["x"], moe_host["idx"], moe_host["w"]
        tokens, top_k = moe_host["tokens"], moe_host["top_k"]
        ym = np.zeros(tokens * 4096, np.float32)
        best, n = best_of(lambda: L.cpub_moe_ffn_batched(E, G, U, D, 12, 12, P(xm), tokens, 4096, 14336, top_k,
                                                         P(idx), P(wts), P(ym)), budget_s, min_reps=2)
        wb = moe_host["weight_bytes"]
        out["config5_moe_mixtral_16tok_top2"] = dict(
            value=round(wb / best / 1e9, 2), unit="GB/s", us=round(best * 1e6, 1), cores=allw, kind="port",
            sample=f"best of {n} MoE steps (16 tokens top-2 over {E} Q4_K experts, the GPU run's routing; per expert "
                   f"the batched SwiGLU via Dispatch, OverfitParallel.For over {allw} workers)", **cpu_meta(L, allw))
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 2000 timed steps of ~38 us (under 0.1 s): a 200-step window still carries start-up effects (~1 % slower)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--copies", type=int, default=4, help="layer copies rotated to defeat the 256 MB cache")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile", choices=["layer", "prefill", "moe", "moe_q6k", "small", "q8", "heads", "config1"],
                    default=None,
                    help="for rocprof runs: only the timed decode-layer loop, the config-3 prefill line, the "
                         "config-5 MoE line (Q4_K or Q6_K down experts), the small-batch layer line, the Q8_0 line, the per-head Q8_0 Wo line "
                         "or the config-1 Q4_K 4096x4096 GEMV line")
    ap.add_argument("--pmc", action="store_true",
                    help="for rocprofv3 --pmc runs: 64 gate/up launches, then 16 plain 64 MiB device copies "
                         "(the counter calibration reference)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the path would shard by output rows across GPUs); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import overfit_amd as ov

    dev = torch.device("cuda:0")
    ctx = ov.default_context()
    copies = [make_layer(ov, torch, 1000 + c) for c in range(args.copies)]
    torch.cuda.synchronize()
    print(f"[bench] built {args.copies} layer copies", file=sys.stderr, flush=True)

    gen = torch.Generator(device="cuda:0").manual_seed(5)
    x_in = {name: torch.randn(k, generator=gen, device=dev) for name, k in
            (("attn", 4096), ("o", 4096), ("ffn", 4096), ("down", 14336))}
    ys = {name: torch.empty(n, device=dev) for name, n, _, _ in LAYER}

    # The step's four C-ABI calls with their pointer arrays built once per layer copy (as a C or C# caller keeps
    # them), so the eager loop measures the library rather than Python's argument conversion.
    def bind_step(ws):
        return (ctx.bind_multi_dev([ws["q"], ws["k"], ws["v"]], x_in["attn"], [ys["q"], ys["k"], ys["v"]]),
                ctx.bind_multi_dev([ws["o"]], x_in["o"], [ys["o"]]),
                ctx.bind_multi_dev([ws["gate"], ws["up"]], x_in["ffn"], [ys["gate"], ys["up"]]),
                ctx.bind_multi_dev([ws["down"]], x_in["down"], [ys["down"]]))

    def step(ws):
        # four launches: each quantises its fp32 activation to Q8_K in-kernel, then runs its projection(s)
        calls = ws.get("_step")
        if calls is None:
            calls = ws["_step"] = bind_step(ws)
        for call in calls:
            call()

    # Warm up eagerly (allocates any scratch), time K eager steps, then also capture one rotation over the layer
    # copies into a HIP graph on a side stream and time its replays (GPU time without Python launch overhead).
    if args.pmc:
        for i in range(64):
            ws = copies[i % len(copies)]
            ctx.project_multi_dev([ws["gate"], ws["up"]], x_in["ffn"], [ys["gate"], ys["up"]])
        torch.cuda.synchronize()
        src = torch.ones(16 * 1024 * 1024, device=dev)  # 64 MiB
        dst = torch.empty_like(src)
        for _ in range(16):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_run": "gate/up x64 then copy 64MiB x16"}), flush=True)
        return

    side = torch.cuda.Stream()

    def capture(calls):
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            ctx.set_stream(side.cuda_stream)
            for fn in calls:  # warm-up on the capture stream
                fn()
            side.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                for fn in calls:
                    fn()
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        return g

    def replay_us(g, n_calls, reps):
        g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * n_calls)

    def gemv_line(n, k, fmt, n_copies, label):
        gen1 = torch.Generator(device="cuda:0").manual_seed(77 + n)
        ws = []
        for _ in range(n_copies):
            wf = torch.randn(n, k, generator=gen1, device=dev) * 0.02
            blocks = ov.quantize_weight(wf, ov.TYPE_Q6_K if fmt == "q6k" else ov.TYPE_Q4_K)
            del wf
            ws.append((ov.Q6KWeight if fmt == "q6k" else ov.Q4KWeight)(blocks, k, n))
            del blocks
        xk = torch.randn(k, generator=gen1, device=dev)
        yk = torch.empty(n, device=dev)
        # at least 16 launches per graph, so the gap between graph replays is not charged to one or two launches
        per_graph = n_copies * max(1, 16 // n_copies)
        g = capture([(lambda w=w: ctx.project_multi_dev([w], xk, [yk])) for w in ws] * (per_graph // n_copies))
        us = replay_us(g, per_graph, max(2, 128 // per_graph))
        nbytes = weight_bytes(n, k, fmt) + 4 * k + 4 * n
        del g, ws
        torch.cuda.empty_cache()
        return {"shape": f"{n}x{k} {fmt}", "avg_us": round(us, 3), "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1),
                "pct_peak": round(100 * nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 2), "algorithmic_bytes": nbytes,
                "copies": n_copies, "what": label}

    def q8_line():
        """Q8_0 projections (the reference's Q8DotKernel path) on a 4096x4096 weight: the decode call (M = 1: the
        persistent decode GEMV, quantising x inside the launch) and M = 512 (Q8_0 quantise + the int8-MFMA kernel),
        graph-replayed over copies past the cache."""
        n = k = 4096
        gen3 = torch.Generator(device="cuda:0").manual_seed(88)
        ws = []
        for _ in range(32):
            wf = torch.randn(n, k, generator=gen3, device=dev) * 0.02
            q, s = ov.quantize_weight(wf, ov.TYPE_Q8_0)
            del wf
            ws.append(ov.Q8Weight(q, s, k, n))
            del q, s
        wbytes = n * k + 4 * (n * k // 32)
        out = {"shape": "4096x4096 q8_0", "weight_bytes": wbytes}
        for m, copies in ((1, 32), (512, 4)):
            x = torch.randn(m * k, generator=gen3, device=dev)
            y = torch.empty(m * n, device=dev)
            per_graph = copies * max(1, 16 // copies)
            g = capture([(lambda w=w: ctx.project_multi_dev([w], x, [y], rows=m)) for w in ws[:copies]]
                        * (per_graph // copies))
            us = replay_us(g, per_graph, max(2, 128 // per_graph))
            del g
            if m == 1:
                nbytes = wbytes + 4 * k + 4 * n
                out["m1"] = {"us": round(us, 3), "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1),
                             "pct_peak": round(100 * nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 2),
                             "what": "decode: one launch, Q8_0 quantisation of x inside the persistent decode GEMV"}
            else:
                tops = 2.0 * m * n * k / (us * 1e-6) / 1e12
                out["m512"] = {"us": round(us, 2), "useful_TOPS": round(tops, 1), "tokens_per_s": round(m / (us * 1e-6), 1),
                               "what": "prefill: Q8_0 quantise of x + the int8-MFMA kernel (one 16x16x32 MFMA per block)"}
        del ws
        torch.cuda.empty_cache()
        out["timing"] = "HIP graph replay over weight copies, per call"
        return out

    def heads_line(n_heads=32, head_dim=128, d_model=4096, n_copies=16):
        """The reference's default Llama decode o-path: Wo requantised per head to Q8_0 (32 heads x [4096][128]),
        output = sum of the head projections in ascending head order, in one launch (ovfq_project_heads_q8_0_dev,
        Q8_0 quantisation inside the launch), graph-replayed over copies past the cache; beside it the same work
        as 32 single-head projection launches (the per-head calls without the fused reduction)."""
        gen5 = torch.Generator(device="cuda:0").manual_seed(55)
        sets = []
        for _ in range(n_copies):
            hs = []
            for _ in range(n_heads):
                wf = torch.randn(d_model, head_dim, generator=gen5, device=dev) * 0.02
                q, s_ = ov.quantize_weight(wf, ov.TYPE_Q8_0)
                del wf
                hs.append(ov.Q8Weight(q, s_, head_dim, d_model))
                del q, s_
            sets.append(hs)
        xh = torch.randn(n_heads * head_dim, generator=gen5, device=dev)
        yh = torch.empty(d_model, device=dev)
        g = capture([(lambda hs=hs: ov.project_heads_q8_0(hs, xh, out=yh)) for hs in sets])
        us = replay_us(g, n_copies, 16)
        del g
        bands = torch.empty(n_heads * d_model, device=dev)
        g = capture([(lambda hs=hs: [ctx.project_dev(hs[h], xh[h * head_dim:(h + 1) * head_dim],
                                                     bands[h * d_model:(h + 1) * d_model])
                                     for h in range(n_heads)]) for hs in sets[:4]])
        us_sep = replay_us(g, 4, 8)
        del g
        # Prefill rows (RT/CachedMultiHeadAttention.cs:689-710): the int8-MFMA kernel (automatic from 9 rows) beside
        # the decode kernel's launches of 8 rows each (forced), graph-replayed over 2 weight copies.
        prefill = {}
        for m in (9, 16, 32, 64, 512):
            xm = torch.randn(m * n_heads * head_dim, generator=gen5, device=dev)
            ym = torch.empty(m * d_model, device=dev)
            calls = [(lambda hs=hs: ov.project_heads_q8_0(hs, xm, rows=m, out=ym)) for hs in sets[:2]] * 2
            g = capture(calls)
            us_m = replay_us(g, 4, 8)
            del g
            ctx.set_batched_kernel("rows")
            g = capture(calls)
            ctx.set_batched_kernel("auto")
            us_8 = replay_us(g, 4, 4)
            del g, xm, ym
            ops = 2.0 * m * d_model * n_heads * head_dim
            prefill["m%d" % m] = {"us": round(us_m, 2), "per8_launches_us": round(us_8, 2),
                                  "useful_TOPS": round(ops / (us_m * 1e-6) / 1e12, 1)}
        del sets
        torch.cuda.empty_cache()
        wb = n_heads * (d_model * head_dim + 4 * d_model * head_dim // 32)
        nbytes = wb + 4 * n_heads * head_dim + 4 * d_model
        return {"what": "Llama-3-8B decode o-projection with per-head Q8_0 Wo (32 x 4096x128), ascending head sum, "
                        "one launch", "us": round(us, 3), "weight_bytes": wb,
                "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1),
                "pct_peak": round(100 * nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 2),
                "separate_launches_us": round(us_sep, 2),
                "prefill": prefill,
                "prefill_what": "the same o-projection over m prefill rows: Q8_0 quantise + the int8-MFMA per-head "
                                "kernel (us) against the decode kernel in launches of 8 rows (per8_launches_us)",
                "timing": "HIP graph replay over %d weight copies, per call (separate: 32 launches, 4 copies; "
                          "prefill: 2 copies)" % n_copies}

    def rows_layer(m):
        """fp32 inputs / outputs for the layer's four projection launches at m rows, and the step over one copy:
        fused q/k/v, o, fused gate/up, down, each quantising its fp32 input to Q8_K first."""
        gen2 = torch.Generator(device="cuda:0").manual_seed(9)
        xp = {name: torch.randn(m * k, generator=gen2, device=dev) for name, k in
              (("attn", 4096), ("o", 4096), ("ffn", 4096), ("down", 14336))}
        yp = {name: torch.empty(m * n, device=dev) for name, n, _, _ in LAYER}

        def pstep(ws):
            ctx.project_multi_dev([ws["q"], ws["k"], ws["v"]], xp["attn"], [yp["q"], yp["k"], yp["v"]], rows=m)
            ctx.project_multi_dev([ws["o"]], xp["o"], [yp["o"]], rows=m)
            ctx.project_multi_dev([ws["gate"], ws["up"]], xp["ffn"], [yp["gate"], yp["up"]], rows=m)
            ctx.project_multi_dev([ws["down"]], xp["down"], [yp["down"]], rows=m)
        return pstep, xp, yp

    def small_batch_line(ms=(2, 4, 8)):
        """Small batches (speculative verification, batched decode): the layer's four projection launches at M
        rows on the automatic kernel choice (multi-row decode / small-M MFMA), graph-replayed over the copies."""
        wb = sum(weight_bytes(n, k, fmt) for _, n, k, fmt in LAYER)
        out = {"what": "Llama-3-8B layer projections (4 launches) at a few activation rows", "weight_bytes": wb,
               "timing": "HIP graph replay over %d layer copies x 4, per layer" % len(copies)}
        for m in ms:
            pstep, xp, yp = rows_layer(m)
            g = capture([(lambda ws=ws: pstep(ws)) for ws in copies] * 4)
            us = replay_us(g, 4 * len(copies), 8)
            del g, xp, yp
            out["m%d" % m] = {"us_per_layer": round(us, 2), "tokens_per_s": round(m / (us * 1e-6), 1),
                              "GB_s": round(wb / (us * 1e-6) / 1e9, 1)}
        torch.cuda.empty_cache()
        return out

    def prefill_line(m=512, n_layers=2):
        """benchmark config 3: the layer's seven projections at M = m rows on the int8-MFMA kernel, in four launches
        (fused q/k/v, o, fused gate/up, down; each quantises its fp32 input to Q8_K first), graph-replayed over
        n_layers weight copies."""
        pstep, xp, yp = rows_layer(m)
        g = capture([(lambda ws=ws: pstep(ws)) for ws in copies[:n_layers]])
        us = replay_us(g, n_layers, 8)
        del g
        ops = 2 * m * sum(n * k for _, n, k, _ in LAYER)
        tops = ops / (us * 1e-6) / 1e12
        # the same layers with the opt-in MFMA-ready copy of every weight (ovfq_weight_prepare_mfma)
        extra = 0
        for ws in copies[:n_layers]:
            for name, n, k, _ in LAYER:
                ws[name].prepare_mfma()
        for name, n, k, fmt in LAYER:
            extra += (n + 63) // 64 * 4 * (k // 256) * 8704 if fmt == "q6k" else 0  # Q4_K: no copy
        g = capture([(lambda ws=ws: pstep(ws)) for ws in copies[:n_layers]])
        us_pre = replay_us(g, n_layers, 8)
        tops_pre = ops / (us_pre * 1e-6) / 1e12
        del g, xp, yp
        torch.cuda.empty_cache()
        roof = lambda t: {"bound": "mfma", "achieved": round(t, 1), "peak": INT8_PEAK_TOPS,  # noqa: E731
                          "unit": "TOPS", "frac": round(t / INT8_PEAK_TOPS, 4),
                          "note": "useful int8 ops 2*M*N*K; the exact kernel issues 2 int8 MFMAs per 64-wide K "
                                  "chunk (lo/hi operand split), plus for Q4_K one fp16 16x16x16 MFMA per super-block "
                                  "and 16-row tile for the min term"}
        return {"what": "benchmark config 3: Llama-3-8B layer projections at M=%d (prefill) on int8 MFMA" % m,
                "us_per_layer": round(us, 2), "tokens_per_s": round(m / (us * 1e-6), 1),
                "useful_TOPS": round(tops, 1), "roofline": roof(tops),
                "prepared_mfma": {"us_per_layer": round(us_pre, 2), "tokens_per_s": round(m / (us_pre * 1e-6), 1),
                                  "useful_TOPS": round(tops_pre, 1), "roofline": roof(tops_pre),
                                  "extra_bytes_per_layer": extra,
                                  "what": "the same launches after ovfq_weight_prepare_mfma on every weight "
                                          "(an MFMA-ready copy of the Q6_K down weight; Q4_K unchanged; "
                                          "bit-identical outputs; GGUF blocks stay resident for decode)"},
                "timing": "HIP graph replay of the 4 launches x %d layer copies, per layer" % n_layers}

    def model_line(n_layers=32):
        """benchmark config 4: one decode token's projections through n_layers distinct Q4_K_M layers plus the
        Q6_K 128256x4096 LM head (RMSNorm / RoPE / attention stay on the host path and are not timed)."""
        layers = copies + [make_layer(ov, torch, 2000 + i) for i in range(n_layers - len(copies))]
        gen3 = torch.Generator(device="cuda:0").manual_seed(4)
        wf = torch.randn(128256, 4096, generator=gen3, device=dev) * 0.02
        head = ov.Q6KWeight(ov.quantize_weight(wf, ov.TYPE_Q6_K), 4096, 128256)
        del wf
        logits = torch.empty(128256, device=dev)

        def token():
            for ws in layers:
                step(ws)
            ctx.project_multi_dev([head], x_in["ffn"], [logits])

        token()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        reps = 5
        e0.record()
        for _ in range(reps):
            token()
        e1.record()
        torch.cuda.synchronize()
        eager_us = e0.elapsed_time(e1) * 1e3 / reps
        g = capture([token])
        graph_us = replay_us(g, 1, 10)
        w = n_layers * layer_algorithmic_bytes()[0] + weight_bytes(128256, 4096, "q6k")
        del g
        host = host_token_line(layers, head)
        del layers[len(copies):], head
        torch.cuda.empty_cache()
        return {"what": "benchmark config 4: %d Llama-3-8B Q4_K_M layers + Q6_K LM head, one decode token, "
                        "projections only (%d launches)" % (n_layers, 4 * n_layers + 1),
                "weight_bytes": w, "eager_us": round(eager_us, 1), "graph_us": round(graph_us, 1),
                "proj_tok_s_eager": round(1e6 / eager_us, 1), "proj_tok_s_graph": round(1e6 / graph_us, 1),
                "GB_s_graph": round(w / (graph_us * 1e-6) / 1e9, 1), "host_pointer_calls": host}

    def host_token_line(layers, head, reps=5):
        """Config 4 end to end through the host-pointer entry points, as the C# drop-in issues them per layer:
        ovfq_project_multi for q/k/v (one quantised hidden row, RT/CachedMultiHeadAttention.cs:196-207), ovfq_project
        for o and ovfq_ffn_swiglu for gate/up -> SiLU*up -> down (RT/CachedFeedForwardBlock.cs:261-318), then the LM
        head: 97 calls per token, each synchronous, its fp32 input copied up from pageable host memory through the
        context's page-locked staging and its outputs copied back. Beside it, the same projections as six separate
        calls per layer (q, k, v, o, gate/up, down; 193 calls). Timed on the host clock around whole tokens; the call
        arguments are prepared ctypes objects, so Python adds about a microsecond per call. Attention, RMSNorm and
        RoPE (host-side by the benchmark's definition) are not run."""
        import ctypes

        lib = ctx.lib
        hx = {k: np.random.default_rng(k).standard_normal(k).astype(np.float32) for k in (4096, 14336)}
        outs = {n: np.zeros(n, np.float32) for n in (4096, 1024, 14336, 128256)}
        qkv = [np.zeros(n, np.float32) for n in (4096, 1024, 1024)]
        up_out = np.zeros(14336, np.float32)
        P = lambda a: ctypes.c_void_p(a.ctypes.data)  # noqa: E731
        x4, x14 = P(hx[4096]), P(hx[14336])
        fused, separate = [], []
        keep = []
        for ws in layers:
            W = (ctypes.c_void_p * 3)(ws["q"].handle.value, ws["k"].handle.value, ws["v"].handle.value)
            Y = (ctypes.c_void_p * 3)(*[a.ctypes.data for a in qkv])
            keep += [W, Y]
            fused.append((lib.ovfq_project_multi, (ctx.handle, 3, W, x4, 1, None, Y)))
            fused.append((lib.ovfq_project, (ctx.handle, ws["o"].handle, x4, 1, None, P(outs[4096]))))
            fused.append((lib.ovfq_ffn_swiglu, (ctx.handle, ws["gate"].handle, ws["up"].handle, ws["down"].handle, x4,
                                                1, P(outs[4096]))))
            for name, n in (("q", 4096), ("k", 1024), ("v", 1024), ("o", 4096)):
                separate.append((lib.ovfq_project, (ctx.handle, ws[name].handle, x4, 1, None, P(outs[n]))))
            separate.append((lib.ovfq_project_gate_up, (ctx.handle, ws["gate"].handle, ws["up"].handle, x4,
                                                        P(outs[14336]), P(up_out))))
            separate.append((lib.ovfq_project, (ctx.handle, ws["down"].handle, x14, 1, None, P(outs[4096]))))
        head_call = (lib.ovfq_project, (ctx.handle, head.handle, x4, 1, None, P(outs[128256])))
        fused.append(head_call)
        separate.append(head_call)

        def best_token_us(calls):
            def token():
                for fn, a in calls:
                    if fn(*a):
                        raise RuntimeError(lib.ovfq_last_error())

            token()
            best = float("inf")
            for _ in range(reps):
                t0 = time.perf_counter()
                token()
                best = min(best, time.perf_counter() - t0)
            return best * 1e6

        us = best_token_us(fused)
        us_sep = best_token_us(separate)
        return {"what": "the same token through the synchronous host-pointer entry points, input up and outputs down "
                        "per call through page-locked staging: q/k/v in one ovfq_project_multi, o, the fused SwiGLU "
                        "FFN, the LM head (%d calls)" % len(fused),
                "us": round(us, 1), "proj_tok_s": round(1e6 / us, 1),
                "separate_calls": {"calls": len(separate), "us": round(us_sep, 1), "proj_tok_s": round(1e6 / us_sep, 1)},
                "timing": "host clock, best of %d tokens" % reps}

    def moe_line(n_sets=2, tokens=16, top_k=2, n_experts=8, keep_host=False, down_fmt="q4k"):
        """benchmark config 5: Mixtral-8x7B-shaped experts (gate/up 14336x4096, down 4096x14336, Q4_K), 16 tokens
        routed top-2 on the device from seeded U[0,1) logits, grouped per-expert SwiGLU; graph-replayed over
        n_sets independent expert sets (> 1.5 GB, past the 256 MB cache). keep_host: also returns host copies of
        the first set's blocks, the tokens and the routing, for the CPU baseline."""
        gen4 = torch.Generator(device="cuda:0").manual_seed(15)
        sets = []
        host = {"gate": [], "up": [], "down": []} if keep_host else None
        for si in range(n_sets):
            mats = {"gate": [], "up": [], "down": []}
            for name in ("gate", "up", "down"):
                n, kk = (4096, 14336) if name == "down" else (14336, 4096)
                q6 = name == "down" and down_fmt == "q6k"
                for _ in range(n_experts):
                    wf = torch.randn(n, kk, generator=gen4, device=dev) * 0.02
                    blocks = ov.quantize_weight(wf, ov.TYPE_Q6_K if q6 else ov.TYPE_Q4_K)
                    mats[name].append((ov.Q6KWeight if q6 else ov.Q4KWeight)(blocks, kk, n))
                    if host is not None and si == 0:
                        host[name].append(blocks.cpu().numpy().reshape(n, -1))
                    del wf, blocks
            sets.append(mats)
        xm = torch.randn(tokens * 4096, generator=gen4, device=dev)
        logits = torch.rand(tokens * n_experts, generator=gen4, device=dev)
        idx = torch.empty(tokens * top_k, dtype=torch.int32, device=dev)
        wts = torch.empty(tokens * top_k, dtype=torch.float32, device=dev)
        ym = torch.empty(tokens * 4096, device=dev)

        def moe_step(m):
            # MoeFeedForwardBlock.DecodeBatched from the router logits: routing inside the grouping launch
            ov.moe_ffn_routed(m["gate"], m["up"], m["down"], xm, tokens, logits, top_k, True, idx, wts, out=ym)

        g = capture([(lambda m=m: moe_step(m)) for m in sets] * 4)  # 8 steps per graph replay
        us = replay_us(g, 4 * n_sets, 10)
        used = len(set(idx.cpu().numpy().tolist()))
        wb = used * (2 * weight_bytes(14336, 4096, "q4k") + weight_bytes(4096, 14336, down_fmt))
        if host is not None:
            host.update(x=xm.cpu().numpy(), idx=idx.cpu().numpy(), w=wts.cpu().numpy(), tokens=tokens,
                        top_k=top_k, weight_bytes=wb)
        del g, sets
        torch.cuda.empty_cache()
        line = {"what": "benchmark config 5: Mixtral-8x7B experts (Q4_K gate/up, %s down), 16 tokens, top-2, one "
                        "MoE step (route + group + quantise in one launch, 2 grouped projections, SwiGLU, the combine "
                        "folded into the down projection: 4 launches)" % ("Q6_K" if down_fmt == "q6k" else "Q4_K"),
                "us": round(us, 1), "experts_used": used, "weight_bytes": wb,
                "GB_s": round(wb / (us * 1e-6) / 1e9, 1), "pct_peak": round(100 * wb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 2),
                "timing": "HIP graph replay of 8 steps over %d expert sets, per step" % n_sets}
        return (line, host) if keep_host else line

    def ffn_line():
        """The fused decode FFN: gate/up -> SiLU*up + Q8_K -> down for one token, 3 launches, over the
        layer copies (the down input is the SwiGLU output, unlike the config-2 step's independent input)."""
        yf = torch.empty(4096, device=dev)
        g = capture([(lambda ws=ws: ov.ffn_swiglu(ws["gate"], ws["up"], ws["down"], x_in["ffn"], 1, out=yf))
                     for ws in copies] * 4)
        us = replay_us(g, 4 * len(copies), 16)
        wb = 2 * weight_bytes(14336, 4096, "q4k") + weight_bytes(4096, 14336, "q6k")
        del g
        return {"what": "fused SwiGLU decode FFN (Llama-3-8B: gate/up Q4_K, down Q6_K), one token, 3 launches",
                "us": round(us, 2), "weight_bytes": wb, "GB_s": round(wb / (us * 1e-6) / 1e9, 1),
                "timing": "HIP graph replay over %d layer copies x 4" % len(copies)}

    if args.profile in ("prefill", "moe", "moe_q6k", "small", "q8", "heads", "config1"):
        only = {"prefill": prefill_line, "moe": moe_line, "moe_q6k": lambda: moe_line(down_fmt="q6k"),
                "small": small_batch_line, "q8": q8_line,
                "heads": heads_line,
                "config1": lambda: gemv_line(4096, 4096, "q4k", 64,
                                             "benchmark config 1: Q4_K 4096x4096 GEMV (quantise in-launch)")}[args.profile]
        print(json.dumps(only()), flush=True)
        return

    for i in range(args.warmup):
        step(copies[i % len(copies)])
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(args.steps):
        step(copies[i % len(copies)])
    t1.record()
    torch.cuda.synchronize()
    eager_ms = t0.elapsed_time(t1) / args.steps

    g_step = capture([(lambda ws=ws: step(ws)) for ws in copies] * 4)  # 16 steps per graph replay
    graph_reps = max(1, args.steps // (4 * len(copies)))
    graph_ms = replay_us(g_step, 4 * len(copies), graph_reps) / 1e3
    ms = eager_ms  # headline: the plain eager loop, exactly K timed steps
    w_bytes, alg_bytes = layer_algorithmic_bytes()
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    if args.profile == "layer":
        print(json.dumps({"ms_per_step": ms, "graph_ms_per_step": graph_ms, "GB/s": gbs}), flush=True)
        return

    # Dominant kernel: the gate/up launch (Q8_K quantise + both 14336x4096 Q4_K GEMVs, 66 MB), replayed from a
    # graph over the layer copies; per-launch time = graph time / launches.
    g_gu = capture([(lambda ws=ws: ctx.project_multi_dev([ws["gate"], ws["up"]], x_in["ffn"], [ys["gate"], ys["up"]]))
                    for ws in copies] * 4)
    gu_avg = replay_us(g_gu, 4 * len(copies), 16)
    gu_bytes = 2 * weight_bytes(14336, 4096, "q4k") + 4 * 4096 + 4 * 2 * 14336
    achieved = gu_bytes / (gu_avg * 1e-6) / 1e9
    traffic = traffic_commit = None
    tfile = os.path.join(ROOT, "profiles", "traffic_q4k_gate_up_gemv.json")
    if os.path.exists(tfile):
        tinfo = json.load(open(tfile))
        traffic, traffic_commit = tinfo.get("bytes_per_launch"), tinfo.get("commit")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "traffic_source": "not measured in this run: the committed profiles/traffic_q4k_gate_up_gemv.json "
                                  "(two rocprofv3 --pmc passes, FETCH_SIZE and WRITE_SIZE, calibrated by a 64 MiB "
                                  "device copy; kernel source of commit %s)" % traffic_commit
                                  if traffic is not None else None,
                "kernel": "kquant_gemv_kernel<Q4K,2,true,4> (Q8_K quantise + fused gate+up GEMV, 2x14336x4096)",
                "avg_us": round(gu_avg, 3), "algorithmic_bytes": gu_bytes,
                "timing": "HIP graph replay of 4x%d launches over %d weight copies, /launch" % (len(copies), len(copies))}

    config1 = gemv_line(4096, 4096, "q4k", 64, "benchmark config 1: Q4_K 4096x4096 GEMV (quantise in-launch)")
    large_q4k = gemv_line(128256, 4096, "q4k", 2, "Q4_K GEMV at LM-head size (asymptotic efficiency)")
    lm_head = gemv_line(128256, 4096, "q6k", 2, "Llama-3-8B Q6_K LM head 128256x4096 (config 4)")
    small = small_batch_line()  # before config 3, which gives the weights their MFMA-ready copies
    config3 = prefill_line()
    config4 = model_line()
    config5, moe_host = moe_line(keep_host=not args.no_cpu_baseline)
    config5_q6k = moe_line(down_fmt="q6k")  # the Q4_K_M layout: Q6_K ffn_down_exps
    ffn = ffn_line()
    q8 = q8_line()
    heads = heads_line()

    cpu = cpu_configs = None
    if not args.no_cpu_baseline:
        host = {name: copies[0][name + "_blocks"].cpu().numpy() for name, _, _, _ in LAYER}
        cpu = run_cpu_baseline(host)
        cpu_configs = run_cpu_configs(host, moe_host)
        del moe_host

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights quantised on device; N(0,1) fp32 activations)",
        "config": {"workload": "llama3-8b layer decode projections, M=1, Q4_K_M mix (benchmark config 2)",
                   "hidden": 4096, "ffn": 14336, "kv_rows": 1024, "formats": "Q4_K q,k,v,o,gate,up + Q6_K down",
                   "weight_bytes_per_step": w_bytes, "algorithmic_bytes_per_step": alg_bytes,
                   "layer_copies_rotated": args.copies},
        "pct_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "decode_proj_tok_s": round(1e3 / ms, 1),
        "graph_ms_per_step": round(graph_ms, 5),
        "timing": "eager loop of K steps between two events (HIP-graph replay of the same steps: graph_ms_per_step)",
        "roofline": roofline,
        "config1_q4k_gemv_4096x4096": config1,
        "config3_prefill_m512": config3,
        "config4_32_layers_lm_head": config4,
        "config5_moe_mixtral_16tok_top2": config5,
        "config5_moe_q6k_down_experts": config5_q6k,
        "ffn_swiglu_decode": ffn,
        "small_batch_layer": small,
        "q4k_gemv_128256x4096": large_q4k,
        "q6k_lm_head_128256x4096": lm_head,
        "q8_0_4096x4096": q8,
        "q8_0_heads_o_proj": heads,
        "cpu_baseline": cpu,
        "cpu_baseline_configs": cpu_configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
