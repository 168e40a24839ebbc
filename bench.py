"""Benchmark of the GGUF quantized-linear decode path on one MI355X.

Workload ("the metric's configuration"): one Llama-3-8B-shaped layer's decode projections
at M = 1 with the Q4_K_M mix — q 4096x4096, k/v 1024x4096, o 4096x4096, gate/up 14336x4096 in Q4_K, down
4096x14336 in Q6_K. Weights N(0, 0.02) from a seed, quantised on the device with the reference quantizer
(GgmlQuant.QuantizeQ4_K) and the library's Q6_K encoder; activations N(0, 1) fp32, resident in HBM.

One step = the layer's four distinct activations quantised to Q8_K and its seven projections:
  quantize(x_attn) + fused q/k/v GEMV, quantize(x_o) + o GEMV, quantize(x_ffn) + fused gate/up GEMV,
  quantize(x_down) + down GEMV.
To measure HBM rather than the 256 MB Infinity Cache, steps rotate over several independent layer copies
(> 2x the cache). value = algorithmic bytes per step / time per step (weights + fp32 activations read once
+ fp32 outputs), in GB/s; decode_proj_tok_s = steps per second.

Also reported: the dominant kernel's roofline (the fused gate/up Q4_K GEMV, per-launch HIP-event timing on
the stream it runs on), BASELINE config 1 (a single Q4_K 4096x4096 GEMV rotated over 64 copies), and the
CPU baseline (the AVX2 C restatement of the reference's CPU path, on a bounded sample, rank 0 only).
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


def run_cpu_baseline(layer0_host, budget_s=2.5):
    """Times the AVX2 C restatement of the reference's decode path on one layer step (7 projections)."""
    import ctypes

    import numpy as np

    import oracle

    L = oracle.lib()
    if not L.cpub_has_avx2():
        return None
    workers = max(1, min(os.cpu_count() or 1, 10))  # OverfitParallel decode cap min(cores, 10)
    L.cpub_set_workers(workers)
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

    step()
    step()
    best = float("inf")
    n = 0
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or n < 3:
        t0 = time.perf_counter()
        step()
        best = min(best, time.perf_counter() - t0)
        n += 1
    _, alg = layer_algorithmic_bytes()
    return {
        "value": round(alg / best / 1e9, 2),
        "unit": "GB/s",
        "tok_s": round(1.0 / best, 2),
        "ms_per_step": round(best * 1e3, 3),
        "cores": workers,
        "kind": "port",
        "sample": f"best of {n} steps of the config-2 layer (7 projections, same Q4_K/Q6_K bytes as the GPU run), "
                  f"AVX2 C restatement of Overfit's CPU path, {workers} row-band workers, ~{budget_s:.1f}s wall",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--copies", type=int, default=4, help="layer copies rotated to defeat the 256 MB cache")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-only", action="store_true", help="only the timed layer loop (for rocprof runs)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the path shards by output rows across GPUs, see "
              "DESIGN.md); run with --gpus 1", file=sys.stderr)
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
    qa = {name: (torch.empty(k, dtype=torch.int8, device=dev), torch.empty(k // 256, device=dev),
                 torch.empty(k // 16, dtype=torch.int16, device=dev)) for name, k in
          (("attn", 4096), ("o", 4096), ("ffn", 4096), ("down", 14336))}

    def step(ws):
        for act, k in (("attn", 4096), ("o", 4096), ("ffn", 4096), ("down", 14336)):
            q, s, b = qa[act]
            ctx.quantize_q8k_dev(x_in[act], 1, k, q, s, b)
        ctx.project_multi_prequantized_dev([ws["q"], ws["k"], ws["v"]], *qa["attn"], [ys["q"], ys["k"], ys["v"]])
        ctx.project_multi_prequantized_dev([ws["o"]], *qa["o"], [ys["o"]])
        ctx.project_multi_prequantized_dev([ws["gate"], ws["up"]], *qa["ffn"], [ys["gate"], ys["up"]])
        ctx.project_multi_prequantized_dev([ws["down"]], *qa["down"], [ys["down"]])

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
    ms = t0.elapsed_time(t1) / args.steps
    w_bytes, alg_bytes = layer_algorithmic_bytes()
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    if args.profile_only:
        print(json.dumps({"ms_per_step": ms, "GB/s": gbs}), flush=True)
        return

    # Dominant kernel: the fused gate/up Q4_K GEMV (66 MB per launch). Per-launch events on the same stream.
    reps = 64
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    q, s, b = qa["ffn"]
    for i in range(reps):
        ws = copies[i % len(copies)]
        ev[i][0].record()
        ctx.project_multi_prequantized_dev([ws["gate"], ws["up"]], q, s, b, [ys["gate"], ys["up"]])
        ev[i][1].record()
    torch.cuda.synchronize()
    gu_us = sorted(a.elapsed_time(c) * 1e3 for a, c in ev)
    gu_avg = sum(gu_us) / len(gu_us)
    gu_bytes = 2 * weight_bytes(14336, 4096, "q4k") + 4 * 4096 + 4 * 2 * 14336
    achieved = gu_bytes / (gu_avg * 1e-6) / 1e9
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "traffic_q4k_gate_up_gemv.json")
    if os.path.exists(tfile):
        traffic = json.load(open(tfile)).get("bytes_per_launch")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "kquant_project_kernel<Q4K> (fused gate+up, 2x14336x4096)",
                "avg_us": round(gu_avg, 3), "median_us": round(gu_us[len(gu_us) // 2], 3),
                "algorithmic_bytes": gu_bytes}

    # Q4_K 4096x4096 GEMV, 64 weight copies (604 MB) rotated.
    gen1 = torch.Generator(device="cuda:0").manual_seed(77)
    c1 = []
    for i in range(64):
        wf = torch.randn(4096, 4096, generator=gen1, device=dev) * 0.02
        c1.append(ov.Q4KWeight(ov.quantize_weight(wf, ov.TYPE_Q4_K), 4096, 4096))
        del wf
    q1, s1, b1 = qa["attn"]
    y1 = torch.empty(4096, device=dev)
    for i in range(8):
        ctx.project_multi_prequantized_dev([c1[i]], q1, s1, b1, [y1])
    ev1 = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(128)]
    for i in range(128):
        ev1[i][0].record()
        ctx.project_multi_prequantized_dev([c1[i % 64]], q1, s1, b1, [y1])
        ev1[i][1].record()
    torch.cuda.synchronize()
    c1_us = sorted(a.elapsed_time(c) * 1e3 for a, c in ev1)
    c1_avg = sum(c1_us) / len(c1_us)
    c1_bytes = weight_bytes(4096, 4096, "q4k") + 4 * 4096 + 4 * 4096
    config1 = {"avg_us": round(c1_avg, 3), "median_us": round(c1_us[len(c1_us) // 2], 3),
               "GB_s": round(c1_bytes / (c1_avg * 1e-6) / 1e9, 1),
               "pct_peak": round(100 * c1_bytes / (c1_avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 2),
               "algorithmic_bytes": c1_bytes, "copies": 64}
    del c1

    cpu = None
    if not args.no_cpu_baseline:
        host = {name: copies[0][name + "_blocks"].cpu().numpy() for name, _, _, _ in LAYER}
        cpu = run_cpu_baseline(host)

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
        "config": {"workload": "llama3-8b layer decode projections, M=1, Q4_K_M mix (BASELINE config 2)",
                   "hidden": 4096, "ffn": 14336, "kv_rows": 1024, "formats": "Q4_K q,k,v,o,gate,up + Q6_K down",
                   "weight_bytes_per_step": w_bytes, "algorithmic_bytes_per_step": alg_bytes,
                   "layer_copies_rotated": args.copies},
        "pct_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "decode_proj_tok_s": round(1e3 / ms, 1),
        "decode_proj_tok_s_32_layers_plus_lm_head_est": None,
        "roofline": roofline,
        "config1_q4k_gemv_4096x4096": config1,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
