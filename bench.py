#!/usr/bin/env python3
"""Benchmark of the MI355X transformer-layer forward (one GPU).

    python bench.py [--steps K] [--warmup W] [--config C2] [--no-cpu-baseline]

A "step" is one forward of the whole layer stack over one batch of
synthetic input (weights: torch.manual_seed(1234) construction; input: CPU
generator seed 1234 + 100000, as the reference harness's timing input,
src/torch_transformer_benchmark.py:529-536), with x already resident in HBM.
W untimed steps, then K steps bracketed by torch.cuda.synchronize(); the
per-step time is the median of per-step HIP-event samples
(src/torch_transformer_benchmark.py:487-499,564).

Prints ONE JSON line.  ``value`` is the per-layer forward latency (median
forward time / num_layers) -- the first component of the baseline metric
"layer fwd latency ms; attn/GEMM % fp16 MFMA peak; LN/epilogue HBM GB/s";
the other two components are reported per kernel under ``kernels`` and,
for the dominant kernel, under ``roofline``.  Per-kernel times come from HIP
events recorded around each launch on the stream the kernel runs on, over a
second pass of K steps.

``cpu_baseline`` times the fp32 CPU oracle (a restatement of the reference's
BaselineTransformer) on this host's cores for a bounded sample of the same
workload.
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import statistics
import sys
import time

REPO = pathlib.Path(__file__).resolve().parent
for _p in (str(REPO), str(REPO / "transformer-kernel_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

METRIC = "layer fwd latency ms; attn/GEMM % fp16 MFMA peak; LN/epilogue HBM GB/s"
PEAK_FP16_TFLOPS = 2516.6  # MI355X dense fp16 MFMA (256 CU x 4096 flop/clk x 2.4 GHz)
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E

# (B, S, D, H, F, L, causal)
CONFIGS = {
    "C1": (64, 128, 128, 4, 128, 4, True),
    "C2": (256, 64, 512, 8, 2048, 4, False),
    "C3": (8, 2048, 1024, 16, 4096, 6, True),
    "C4": (4, 8192, 2048, 16, 8192, 2, True),
    "C5": (2, 32768, 1024, 16, 4096, 1, True),
}


def cpu_cores() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        n = min(n, int(env))
    return max(1, n)


def kernel_units(name: str, cfg) -> tuple:
    """(algorithmic amount per launch, unit, bound) for a kernel role."""
    b, s, d, h, f, _, causal = cfg
    t = b * s
    gemm = {
        "qkv": 2.0 * t * 3 * d * d,
        "out_proj_ln": 2.0 * t * d * d,
        "out_proj_resid": 2.0 * t * d * d,
        "ffn_up_gelu": 2.0 * t * f * d,
        "ffn_down_ln": 2.0 * t * d * f,
        "ffn_down_resid": 2.0 * t * d * f,
    }
    if name in gemm:
        return gemm[name], "flop", "mfma"
    if name == "flash_attn":
        pairs = s * (s + 1) / 2 if causal else s * s
        return 4.0 * b * d * pairs, "flop", "mfma"
    ln_bytes = {"ln_in": 6, "ln2": 6, "ln_next": 6, "ln_final": 8}
    if name in ln_bytes:
        return float(ln_bytes[name] * t * d), "byte", "hbm"
    raise KeyError(name)


COPY_BYTES = 512 * 1024 * 1024  # per direction


def copy_calibration() -> int:
    """Ten plain copies of COPY_BYTES (read COPY_BYTES, write COPY_BYTES each)."""
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_direction": COPY_BYTES, "launches": 10}), flush=True)
    return 0


def measured_traffic(config: str, kernel: str):
    """HBM bytes per launch of ``kernel`` at ``config`` from the committed rocprofv3
    FETCH_SIZE + WRITE_SIZE summary (profiles/traffic.json), or None."""
    path = REPO / "profiles" / "traffic.json"
    try:
        table = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    entry = table.get("kernels", {}).get(config, {}).get(kernel)
    return None if entry is None else entry.get("bytes_per_launch")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C2", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-check", action="store_true", help="skip the one-trial parity check")
    ap.add_argument("--graph", action="store_true",
                    help="time the whole forward replayed from a HIP graph (tkmi.graphs.GraphedTransformer)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of COPY_BYTES (torch copy_), the reference kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    ap.add_argument("--unfused-norm", action="store_true",
                    help="residual GEMM + standalone LayerNorm instead of the fused GEMM+LN epilogue")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one GPU only: this build has no multi-GPU path "
            "(see the sharding section of DESIGN.md); run with --gpus 1",
            file=sys.stderr,
        )
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X)", file=sys.stderr)
        return 2

    if args.copy_calibration:
        return copy_calibration()

    import tkmi
    from tkmi import ops
    from oracle import baseline as ob  # parity check and cpu_baseline only

    cfg_t = CONFIGS[args.config]
    b, s, d, h, f, nl, causal = cfg_t
    cfg = ob.TransformerConfig(b, s, d, h, f, nl, causal)
    dev = torch.device("cuda:0")
    torch.set_num_threads(cpu_cores())
    torch.set_float32_matmul_precision("highest")

    base = ob.build_model(cfg, seed=1234).eval()
    settings = tkmi.OptimizerSettings(fused_norm=not args.unfused_norm)
    model = tkmi.OptimizedTransformer(tkmi.TransformerConfig(*cfg_t), settings)
    ob.copy_model_weights(base, model, strict=True)
    model = model.to(dev).eval()
    timed_model = model
    if args.graph:
        from tkmi.graphs import GraphedTransformer

        timed_model = GraphedTransformer(tkmi.TransformerConfig(*cfg_t), settings)
        ob.copy_model_weights(base, timed_model, strict=True)
        timed_model = timed_model.to(dev).eval()

    parity = None
    if not args.no_check and args.config in ("C1", "C2"):
        x_chk, m_chk = ob.generate_random_case(cfg, seed=1234)
        with torch.inference_mode():
            got = model(x_chk.to(dev), m_chk.to(dev)).cpu()
            ref = base(x_chk, m_chk)
        r = ob.compare_outputs(ref, got)
        parity = {"passed": r.passed, "max_abs": r.max_abs_error, "failed": r.failed_elements,
                  "elements": r.total_elements, "trial_seed": 1234}
        print(f"[bench] parity {args.config}: {'PASS' if r.passed else 'FAIL'} max_abs={r.max_abs_error:.3g}",
              file=sys.stderr, flush=True)
        del x_chk, m_chk, got, ref

    x, mask = ob.generate_random_case(cfg, seed=1234 + 100000)
    x, mask = x.to(dev), mask.to(dev)

    with torch.inference_mode():
        for _ in range(max(args.warmup, 10 if args.graph else 0)):
            timed_model(x, mask)
        torch.cuda.synchronize()
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
        t0 = time.perf_counter()
        for i in range(args.steps):
            starts[i].record()
            timed_model(x, mask)
            ends[i].record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        samples = [a.elapsed_time(e) for a, e in zip(starts, ends)]
        print(f"[bench] timed {args.steps} steps in {wall:.3f}s", file=sys.stderr, flush=True)

        # Per-kernel durations: events around each launch, on the launch stream.
        with ops.kernel_timer() as rec:
            for _ in range(args.steps):
                model(x, mask)
            torch.cuda.synchronize()
        per = {}
        for name, e0, e1 in rec:
            per.setdefault(name, []).append(e0.elapsed_time(e1))

    fwd_ms = statistics.median(samples)
    kernels = {}
    for name, ts in per.items():
        amount, unit, bound = kernel_units(name, cfg_t)
        avg_ms = sum(ts) / len(ts)
        rate = amount / (avg_ms * 1e-3)
        if bound == "mfma":
            ach, peak, u = rate / 1e12, PEAK_FP16_TFLOPS, "TFLOP/s"
        else:
            ach, peak, u = rate / 1e9, PEAK_HBM_GBPS, "GB/s"
        kernels[name] = {
            "avg_ms": round(avg_ms, 5),
            "launches_per_step": len(ts) // args.steps,
            "ms_per_step": round(sum(ts) / args.steps, 5),
            "bound": bound,
            "achieved": round(ach, 2),
            "unit": u,
            "frac": round(ach / peak, 4),
            "algorithmic_per_launch": amount,
            "algorithmic_unit": unit,
        }
    dom_name = max(kernels, key=lambda k: kernels[k]["ms_per_step"])
    dom = kernels[dom_name]
    roofline = {
        "kernel": dom_name,
        "bound": dom["bound"],
        "achieved": dom["achieved"],
        "peak": PEAK_FP16_TFLOPS if dom["bound"] == "mfma" else PEAK_HBM_GBPS,
        "unit": dom["unit"],
        "frac": dom["frac"],
        "traffic": measured_traffic(args.config, dom_name),
    }

    cpu = None
    if not args.no_cpu_baseline:
        cores = cpu_cores()
        torch.set_num_threads(cores)
        if args.config in ("C4", "C5"):
            sample_b = 1
            xs, _ = ob.generate_random_case(ob.TransformerConfig(1, s, d, h, f, nl, causal), seed=101234)
            fn = lambda t: ob.chunked_forward(base, t, q_chunk=2048)  # noqa: E731
            sample = f"query-chunked fp32 oracle, batch 1 of {b}, x{b} scaled; 1 repeat after 0 warmup"
            reps, warm = 1, 0
        else:
            sample_b = b
            xs = x.cpu()
            fn = None
            sample = f"full {args.config} forward (B{b} S{s}), median of 3 after 1 warmup"
            reps, warm = 3, 1
        ts = ob.time_cpu_forward(base, xs, warmup=warm, repeats=reps, fn=fn)
        cpu_fwd = statistics.median(ts) * (b / sample_b)
        cpu = {
            "value": round(cpu_fwd / nl, 3),
            "unit": "ms",
            "cores": cores,
            "kind": "port",
            "sample": sample,
            "forward_ms": round(cpu_fwd, 2),
        }

    t = b * s
    line = {
        "metric": METRIC,
        "value": round(fwd_ms / nl, 5),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(fwd_ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 operands, fp32 accumulate / residual / statistics",
        "data": "synthetic (seeded randn input, seeded nn.Linear default init)",
        "config": {
            "workload": f"{args.config}: B{b} S{s} D{d} H{h} F{f} L{nl} {'causal' if causal else 'non-causal'}",
            "batch": b, "seq_len": s, "d_model": d, "heads": h, "ffn_dim": f, "layers": nl,
            "causal": causal, "parallelism": "single GPU", "fused_norm": not args.unfused_norm,
            "hip_graph": bool(args.graph),
        },
        "tokens_per_s": round(t * 1000.0 / fwd_ms, 1),
        "wall_s_timed": round(wall, 4),
        "roofline": roofline,
        "kernels": kernels,
        "cpu_baseline": cpu,
        "parity": parity,
        "device": torch.cuda.get_device_name(0),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
