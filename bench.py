#!/usr/bin/env python3
"""Hybrid-block prefill benchmark on one MI355X.

A step is one prefill of the hybrid block stack (3 gated-DeltaNet layers and
1 gated GQA attention layer, hidden 2048, SwiGLU 6144, DeltaNet heads 16/32 x
128, attention 16q/2kv x 256, rotary on 64 dims; weights ~ N(0, 0.02), seed
3) over T = 4096 token ids (uniform in [0, 151936)), in the mixed-f16 profile
(f16 projections with f32 accumulation, f32 residual stream, f16-MFMA scan
with f32 state).  Inputs and weights are resident in HBM before timing.

The JSON line reports whole-prefill tokens/s, the projection GEMMs' TFLOP/s
and the scan's fraction of the HBM roofline (both from HIP events recorded on
the prefill's stream around each launch), the stand-alone scan of the full
layer shape (T=4096, Hk=16, Hv=32, 128/128, f16 in, f32 out) in both
precision profiles, the projection GEMMs at the 2048 x 2048 shapes in f16 and
f32, the same block in the f32 profile, and the CPU oracle on bounded
samples of the same workloads.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "clef-rs_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFS = {"f16": 2500.0, "f32": 157.3}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--tokens", type=int, default=4096)
    ap.add_argument("--profile", choices=("mixed", "f32"), default="mixed")
    ap.add_argument("--cpu-tokens", type=int, default=2048,
                    help="tokens of the bounded CPU-oracle sample (0 disables it)")
    ap.add_argument("--cpu-runs", type=int, default=3, help="timed CPU runs (median) after one warm-up")
    ap.add_argument("--sweep", type=int, default=1,
                    help="also time the 2048 x 2048 projection GEMMs (f16 and f32), the stand-alone scan in "
                         "both profiles and the block in the f32 profile (0: skip)")
    ap.add_argument("--ragged", type=int, default=1,
                    help="also time the ragged batch: 32 requests of U[128, 4096] tokens behind one shared "
                         "512-token prefix (0: skip)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="first run one plain device copy of this many MiB (the known-size reference for "
                         "HBM byte counters under rocprofv3 --pmc)")
    ap.add_argument("--only", choices=("gemm", "gemm_vendor", "attention", "scan", "ragged"), default=None,
                    help="run five calls of one kernel workload and exit (for counter profiles): the f16 "
                         "projection GEMM (default 4096 x 12288 x 2048), the same product through "
                         "torch.matmul (the vendor BLAS, for a side-by-side profile), the attention core at "
                         "T=4096 (16 q / 2 kv heads, d=256), the full-layer scan (mixed profile), or the "
                         "ragged prefill (32 requests behind a 512-token prefix, mixed profile)")
    ap.add_argument("--gemm-shape", default="4096,12288,2048",
                    help="M,N,K of --only gemm / gemm_vendor (y[M,N] = x[M,K] . W[N,K]^T, f16 in and out)")
    return ap.parse_args()


def only_workload(name, torch, gemm_shape="4096,12288,2048"):
    """Five calls of one kernel on seeded inputs, nothing else on the GPU:
    the program a rocprofv3 counter pass of that kernel runs."""
    import clef_hip
    import workloads
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(7)
    if name in ("gemm", "gemm_vendor"):
        M, N, K = (int(v) for v in gemm_shape.split(","))
        x, w = workloads.gemm_inputs(1, M, N, K, dtype=torch.float16, device=dev)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        if name == "gemm":
            fn = lambda: clef_hip.gemm(x, w, out=y)
        else:  # the same product on the vendor BLAS (hipBLASLt under torch.matmul)
            wt = w.t()
            fn = lambda: torch.matmul(x, wt, out=y)
    elif name == "attention":
        T, H, KV, d = 4096, 16, 2, 256
        q = torch.randn((H, T, d), generator=gen, device=dev).half()
        k = torch.randn((KV, T, d), generator=gen, device=dev).half()
        vt = torch.randn((KV, d, T), generator=gen, device=dev).half()
        gate = torch.randn((T, H, d), generator=gen, device=dev).half()
        fn = lambda: clef_hip.attention_gated(q, k, vt, gate)
    elif name == "ragged":
        import numpy as np
        cfg = workloads.block_config()
        model = clef_hip.Backbone(cfg, workloads.block_weights(cfg, seed=3, device=dev), profile="mixed",
                                  max_tokens=512 + 4096)
        prefix_ids, lens, req_ids, cu = workloads.ragged_workload(cfg, seed=4)
        _, state = model.prefill(np.concatenate([prefix_ids, req_ids[:1]]), capture=512)
        hidden = torch.empty((int(lens.sum()), cfg["hidden_size"]), dtype=torch.float32, device=dev)
        fn = lambda: model.prefill_varlen(req_ids, cu, initial=state, hidden=hidden)
    else:
        q, k, v, g, beta = workloads.scan_inputs(2, 4096, 16, 32, 128, 128, dtype=torch.float16, device=dev)
        out = torch.empty((4096, 32, 128), device=dev)
        scan = clef_hip.DeltaScan(128, 128, "mixed")
        fn = lambda: scan.prefill(q, k, v, g, beta, out=out, want_final=True)
    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    print(json.dumps({"only": name, "calls": 5}), flush=True)


def measured_traffic(T, profile):
    """HBM bytes per GEMM launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a copy of known size) and
    that summary's path, or (None, None) when no summary matches this
    workload.  Counters need a profiler run of their own, so this is the
    committed measurement of the same workload, not one taken in this run."""
    path = ROOT / "profiles" / f"gemm_traffic_T{T}_{profile}.md"
    if not path.exists():
        return None, None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch"):
            return int(float(line.split("=")[1])), str(path.relative_to(ROOT))
    return None, None


def event_ms(fn, steps, warmup, torch):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def cpu_baseline(cfg, weights, ids, tokens, runs):
    """Times the oracle (C restatement of the reference CPU F32 path) on the
    first `tokens` ids of the same workload; only the gathered embedding rows
    are copied to the host."""
    import numpy as np
    import torch

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle  # CPU baseline leg only

    sample = ids[:tokens]
    uniq, inv = np.unique(sample, return_inverse=True)
    emb_name = "model.language_model.embed_tokens.weight"
    host = {k: v.float().cpu().numpy() for k, v in weights.items() if k != emb_name}
    host[emb_name] = weights[emb_name][torch.from_numpy(uniq).long().to(weights[emb_name].device)].float().cpu().numpy()
    b = oracle.Backbone(dict(cfg, vocab_size=len(uniq)), host)
    med, total = _median_after_warmup(lambda: b.prefill(inv.astype(np.int32)), runs)
    out = {"value": round(tokens / med, 2), "unit": "tok/s", "cores": oracle.threads(), "kind": "port",
           "sample": f"oracle F32 prefill of the first {tokens} tokens of the same block workload "
                     f"(same weights), median of {runs} runs after one warm-up ({total:.1f} s in all)"}
    out["ops"] = cpu_ops(runs)
    return out


def _median_after_warmup(fn, runs):
    t_all = time.perf_counter()
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], time.perf_counter() - t_all


def cpu_ops(runs):
    """The oracle's scan at the small (T=256, H=4, 64/64) and full layer
    shapes and one 2048 x 2048 x 8192 projection, beside the GPU figures."""
    import numpy as np
    import torch

    import oracle  # CPU baseline leg only
    import workloads

    res = {}
    for name, shape in (("scan_T256_H4_64", workloads.SCAN_SMALL), ("scan_T4096_16x32_128", workloads.SCAN_LAYER)):
        q, k, v, g, beta = (x.numpy() for x in workloads.scan_inputs(**shape, device="cpu"))
        n = 1 if shape["T"] > 1024 else runs
        med, _ = _median_after_warmup(lambda: oracle.delta_scan(q, k, v, g, beta), n)
        res[name + "_ms"] = round(med * 1e3, 2)
    x, w = (t.float().numpy() for t in workloads.gemm_inputs(1, 2048, 8192, 2048, dtype=torch.float32,
                                                              device="cpu"))
    med, _ = _median_after_warmup(lambda: oracle.linear(x, w), runs)
    res["gemm_2048x8192x2048_ms"] = round(med * 1e3, 2)
    res["gemm_2048x8192x2048_tfs"] = round(2 * 2048 * 8192 * 2048 / med / 1e12, 4)
    return res


def gemm_sweep(clef_hip, workloads, torch, dev, steps, warmup):
    """The projection GEMMs at M = K = 2048 (N = 8192 fused in-projection,
    2048 out-projection, 6144 SwiGLU gate + up), x ~ N(0,1), W ~ N(0,0.02),
    seed 1, f16 and f32 operands, f32 accumulation; HIP events on the
    launching stream, outputs preallocated."""
    rows = []
    for dt, name in ((torch.float16, "f16"), (torch.float32, "f32")):
        peak = MFMA_PEAK_TFS[name]
        for label, N in (("in_proj", 8192), ("out_proj", 2048), ("swiglu", 6144)):
            x, w = workloads.gemm_inputs(1, 2048, N, 2048, dtype=dt, device=dev)
            y = torch.empty((2048, N), dtype=dt, device=dev)
            if label == "swiglu":
                _, wu = workloads.gemm_inputs(2, 2048, N, 2048, dtype=dt, device=dev)
                fn = lambda: clef_hip.gemm_swiglu(x, w, wu, out=y)
                flops = 4.0 * 2048 * N * 2048
            else:
                fn = lambda: clef_hip.gemm(x, w, out=y)
                flops = 2.0 * 2048 * N * 2048
            ms = event_ms(fn, steps, warmup, torch)
            tfs = flops / (ms * 1e-3) / 1e12
            rows.append({"dtype": name, "shape": f"2048x{N}x2048" + (" x2 (gate+up)" if label == "swiglu" else ""),
                         "op": label, "us": round(ms * 1e3, 2), "tflops": round(tfs, 2), "frac": round(tfs / peak, 4)})
    return rows


def scan_standalone(clef_hip, workloads, torch, dev, steps, warmup):
    """The full-layer scan (T=4096, Hk=16, Hv=32, 128/128, seed 2; f16 q/k/v/g/beta,
    f32 state and output) in the mixed (f16 MFMA) and strict (f32 MFMA) profiles."""
    q, k, v, gg, beta = workloads.scan_inputs(2, 4096, 16, 32, 128, 128, dtype=torch.float16, device=dev)
    sout = torch.empty((4096, 32, 128), device=dev)
    sbytes = workloads.scan_bytes(4096, 16, 32, 128, 128, 2, 4)
    sflops = workloads.scan_flops(4096, 16, 32, 128, 128)
    out = {}
    for prec, peak_name in (("mixed", "f16"), ("strict", "f32")):
        scan = clef_hip.DeltaScan(128, 128, prec)
        sms = event_ms(lambda: scan.prefill(q, k, v, gg, beta, out=sout, want_final=True), steps, warmup, torch)
        gbs = sbytes / (sms * 1e-3) / 1e9
        out[prec] = {"us": round(sms * 1e3, 2), "GBs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                     "tflops": round(sflops / (sms * 1e-3) / 1e12, 2),
                     "frac_mfma": round(sflops / (sms * 1e-3) / 1e12 / MFMA_PEAK_TFS[peak_name], 4)}
    out["algorithmic_bytes"] = sbytes
    out["algorithmic_flops"] = sflops
    return out


def ragged_batch(model, cfg, args, torch, np, dev):
    """32 packed requests (lengths uniform in [128, 4096], seed 4) resumed
    from one shared 512-token prefix whose per-layer DeltaNet states, conv
    history and attention K/V are computed once, before timing; a step is one
    ragged prefill of all requests (cu_seqlens packing, each request with its
    own state and causal mask)."""
    import workloads
    prefix_ids, lens, req_ids, cu = workloads.ragged_workload(cfg, seed=4)
    _, state = model.prefill(np.concatenate([prefix_ids, req_ids[:1]]), capture=512)
    hidden = torch.empty((int(lens.sum()), cfg["hidden_size"]), dtype=torch.float32, device=dev)
    ms = event_ms(lambda: model.prefill_varlen(req_ids, cu, initial=state, hidden=hidden), args.steps,
                  args.warmup, torch)
    return {"workload": "32 requests, lengths uniform in [128, 4096] (seed 4), one shared 512-token prefix "
                        "computed once; cu_seqlens packing", "tokens": int(lens.sum()), "prefix": 512,
            "ms_per_step": round(ms, 4), "tok_s": round(int(lens.sum()) / (ms / 1e3), 1)}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: there is no multi-GPU path "
              "(the scan would shard over v-heads and the GEMMs over columns). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import clef_hip
    import workloads

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_mib > 0:
        src = torch.ones(args.copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.only:
        only_workload(args.only, torch, args.gemm_shape)
        return
    T = args.tokens
    cfg = workloads.block_config()
    weights = workloads.block_weights(cfg, seed=3, device=dev)
    ids = workloads.block_ids(cfg, T, seed=3).numpy()
    # max_tokens bounds prefix + request length (the ragged batch reaches 512 + 4096)
    model = clef_hip.Backbone(cfg, weights, profile=args.profile, max_tokens=max(8192, T))
    hidden = torch.empty((T, cfg["hidden_size"]), dtype=torch.float32, device=dev)

    # ---- timed region: whole prefills
    step = lambda: model.prefill(ids, hidden=hidden)
    ms = event_ms(step, args.steps, args.warmup, torch)
    value = T / (ms / 1e3)

    # ---- same steps with per-launch events (categories and roofline)
    model.enable_timing(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    cats = model.timings()
    model.enable_timing(False)
    per_step = {k: {kk: vv / args.steps for kk, vv in v.items()} for k, v in cats.items()}
    dt = "f16" if args.profile == "mixed" else "f32"
    g = per_step["gemm"]
    gemm_tfs = g["flops"] / (g["ms"] * 1e-3) / 1e12
    sc = per_step["scan"]
    scan_gbs = sc["bytes"] / (sc["ms"] * 1e-3) / 1e9

    # ---- stand-alone scan at the full layer shape (f16 in, f32 state and out)
    scans = scan_standalone(clef_hip, workloads, torch, dev, args.steps, args.warmup)
    sprof = scans["mixed" if args.profile == "mixed" else "strict"]
    traffic, traffic_src = measured_traffic(T, args.profile)

    line = {
        "metric": "prefill tok/s (hybrid block, T=4096); GEMM TFLOP/s + scan % of HBM roofline",
        "value": round(value, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dt,
        "data": "synthetic (seeded random-init weights N(0,0.02), uniform token ids)",
        "config": {
            "workload": f"hybrid block prefill: 3 gated-DeltaNet + 1 gated GQA attention layer, hidden 2048, "
                        f"SwiGLU 6144, T={T}, " + (
                            "mixed-f16 profile (f16 projection operands, f32 accumulation and residual; the "
                            "scan on f16 MFMA with f32 accumulation, its f32 state rounded to f16 as the "
                            "products' operand each chunk)" if dt == "f16" else "f32 profile"),
            "tokens": T, "global_batch": 1, "seq_len": T, "layers": 4,
        },
        "roofline": {
            "kernel": "projection GEMMs (gemm_f16_w4 / gemm_f16_dma / gemm_kernel, all launches of a step)",
            "bound": "mfma",
            "achieved": round(gemm_tfs, 2),
            "peak": MFMA_PEAK_TFS[dt],
            "unit": "TFLOP/s",
            "frac": round(gemm_tfs / MFMA_PEAK_TFS[dt], 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            # per launch (event-timed on the backbone's stream), to set beside
            # the kernel-trace averages
            "launches_per_step": int(g["launches"]),
            "avg_launch_us": round(g["ms"] * 1e3 / g["launches"], 2),
            "flops_per_launch": g["flops"] / g["launches"],
        },
        "scan": {
            "in_block_GBs": round(scan_gbs, 1),
            "in_block_frac_hbm": round(scan_gbs / HBM_PEAK_GBS, 4),
            "layer_shape_us": sprof["us"],
            "layer_shape_GBs": sprof["GBs"],
            "layer_shape_frac_hbm": sprof["frac_hbm"],
            "algorithmic_bytes": scans["algorithmic_bytes"],
            "layer_shape_by_profile": {k: v for k, v in scans.items() if k in ("mixed", "strict")},
        },
        "breakdown_ms_per_step": {k: round(v["ms"], 4) for k, v in per_step.items()},
        "launches_per_step": {k: int(v["launches"]) for k, v in per_step.items()},
    }
    if args.ragged:
        line["ragged"] = ragged_batch(model, cfg, args, torch, np, dev)
    if args.sweep:
        line["gemm_2048"] = gemm_sweep(clef_hip, workloads, torch, dev, args.steps, args.warmup)
        if args.profile == "mixed":
            # the reference's own mixed profile: f16 projections, the whole
            # recurrence in f32 (qwen.rs:843-848)
            mref = clef_hip.Backbone(cfg, weights, profile="mixed", scan_precision="strict",
                                     max_tokens=max(8192, T))
            msr = event_ms(lambda: mref.prefill(ids, hidden=hidden), args.steps, args.warmup, torch)
            line["mixed_f16_gemm_f32_scan"] = {
                "tok_s": round(T / (msr / 1e3), 1), "ms_per_step": round(msr, 4), "steps": args.steps,
                "profile": "f16 projections with f32 accumulation, scan in f32 on f32 MFMA (the reference's "
                           "mixed profile: the recurrence stays f32)"}
            del mref, model
            torch.cuda.empty_cache()
            m32 = clef_hip.Backbone(cfg, weights, profile="f32", max_tokens=max(8192, T))
            ms32 = event_ms(lambda: m32.prefill(ids, hidden=hidden), max(2, args.steps // 3), 1, torch)
            line["f32_profile"] = {"tok_s": round(T / (ms32 / 1e3), 1), "ms_per_step": round(ms32, 3),
                                   "steps": max(2, args.steps // 3)}
            del m32
    if args.cpu_tokens > 0:
        line["cpu_baseline"] = cpu_baseline(cfg, weights, ids, min(args.cpu_tokens, T), args.cpu_runs)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
