#!/usr/bin/env python3
"""Benchmark of the MI355X transformer-layer forward (one GPU).

    python bench.py [--steps K] [--warmup W] [--config C4] [--no-cpu-baseline]
    python bench.py --shape 64,128,128,4,128,4,causal [--dtype float16]

A "step" is one forward of the whole layer stack over one batch of
synthetic input (weights: torch.manual_seed(1234) construction of the
module tree, src/torch_transformer_benchmark.py:683-699; input: CPU
generator seed 1234 + 100000, as the reference harness's timing input,
src/torch_transformer_benchmark.py:529-536), with x already resident in HBM.
``--shape B,S,D,H,F,L[,causal]`` times any shape; ``--dtype`` sets the model
and input dtype as the harness's --dtype does
(src/torch_transformer_benchmark.py:609-613, 698-699).
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

The default workload is C4 (B4 S8192 D2048 H16 F8192 L2, causal), the
largest BASELINE.json configuration by work per forward (8.8 TFLOP); the
other configurations run with ``--config``.

``cpu_baseline`` times the fp32 CPU oracle (a restatement of the reference's
BaselineTransformer) on this host's cores for a bounded sample of the same
workload: the whole forward for C1-C3-sized shapes, one sequence of the batch
through the query-chunked oracle (row-exact to the baseline, without the
[B, H, S, S] score tensor) for C4/C5-sized ones.  The sample's output also
checks the GPU forward's rows it covers (``parity``, the harness's element
rule).  The oracle is used by that leg only.
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
INFINITY_CACHE_BYTES = 256 * 1024 * 1024  # MI355X last-level (MALL) cache

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


def kernel_units(name: str, cfg) -> dict:
    """Algorithmic work of one launch of a kernel role: {"flop": F, "byte": B}.

    Each unit present is priced against its roof (fp16 MFMA peak, HBM
    bandwidth); the role is bound by whichever roof takes longer.  Bytes are
    the launch's compulsory HBM traffic: every operand read once and every
    output written once (fp16 GEMM operands and outputs 2 B/element, an fp32
    residual read 4 + sum write 4 B/element, the fused residual + LayerNorm
    epilogue 4 + 4 + 2).
    """
    b, s, d, h, f, nl, causal = cfg
    t = b * s
    pairs = s * (s + 1) / 2 if causal else s * s
    # (M, N, K, output bytes per element) of each GEMM role
    gemm = {
        "qkv": (t, 3 * d, d, 2),
        "out_proj_ln": (t, d, d, 10),
        "out_proj_resid": (t, d, d, 8),
        "ffn_up_gelu": (t, f, d, 2),
        "ffn_down_ln": (t, d, f, 10),
        "ffn_down_resid": (t, d, f, 8),
    }
    if name in gemm:
        m, n, k, ob = gemm[name]
        return {"flop": 2.0 * m * n * k, "byte": 2.0 * (m * k + n * k) + 4.0 * n + float(ob) * m * n}
    if name == "small_forward":  # the whole forward (every layer) in one launch
        per_layer = 2.0 * t * (3 * d * d + d * d + 2 * d * f) + 4.0 * b * d * pairs
        return {"flop": per_layer * nl}
    if name == "qkv_attn":  # fused QKV projection + one-tile attention: h and W in, ctx out
        return {"flop": 2.0 * t * 3 * d * d + 4.0 * b * d * pairs, "byte": 2.0 * t * d * 2 + 2.0 * 3 * d * d}
    if name == "flash_attn":  # Q, K, V read and the context written once (fp16)
        return {"flop": 4.0 * b * d * pairs, "byte": 8.0 * t * d}
    ln_bytes = {"ln_in": 6, "ln2": 6, "ln_next": 6, "ln_final": 8}
    if name in ln_bytes:
        return {"byte": float(ln_bytes[name] * t * d)}
    raise KeyError(name)


def kernel_roofline(name: str, cfg, avg_ms: float) -> dict:
    """Both roofline fractions of a role's average launch and the binding one."""
    units = kernel_units(name, cfg)
    secs = avg_ms * 1e-3
    out = {}
    if "flop" in units:
        out["flop_per_launch"] = units["flop"]
        out["frac_mfma"] = round(units["flop"] / secs / (PEAK_FP16_TFLOPS * 1e12), 4)
    if "byte" in units:
        out["bytes_per_launch"] = units["byte"]
        out["frac_hbm"] = round(units["byte"] / secs / (PEAK_HBM_GBPS * 1e9), 4)
    t_mfma = units.get("flop", 0.0) / (PEAK_FP16_TFLOPS * 1e12)
    t_hbm = units.get("byte", 0.0) / (PEAK_HBM_GBPS * 1e9)
    if t_mfma >= t_hbm:
        out.update(bound="mfma", achieved=round(units["flop"] / secs / 1e12, 2), unit="TFLOP/s",
                   frac=out["frac_mfma"], algorithmic_per_launch=units["flop"], algorithmic_unit="flop")
    else:
        out.update(bound="hbm", achieved=round(units["byte"] / secs / 1e9, 2), unit="GB/s",
                   frac=out["frac_hbm"], algorithmic_per_launch=units["byte"], algorithmic_unit="byte")
    return out


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


# GEMM roles of one layer: (M, N, K, epilogue) for a config
def gemm_roles(cfg) -> dict:
    b, s, d, h, f, _, _ = cfg
    t = b * s
    return {"qkv": (t, 3 * d, d, "bias"), "out_proj_resid": (t, d, d, "resid"),
            "ffn_up_gelu": (t, f, d, "gelu"), "ffn_down_resid": (t, d, f, "resid")}


def gemm_yardstick(configs, reps: int) -> int:
    """Time this build's GEMM and hipBLASLt (through torch's F.linear, a plain
    fp16 GEMM + fp16 bias) on every GEMM role of the given configs, same
    process, same buffers.  One JSON line per role; run it under
    ``rocprofv3 --kernel-trace --stats`` for the library's kernel names and
    durations.  hipBLASLt is a yardstick only: it is never on the forward
    path."""
    import torch.nn.functional as F
    from tkmi import ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cpu").manual_seed(5)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for e0, e1 in ev:
            e0.record()
            fn()
            e1.record()
        torch.cuda.synchronize()
        return statistics.median(e0.elapsed_time(e1) for e0, e1 in ev)

    for name in configs:
        cfg = CONFIGS[name]
        for role, (m, n, k, epi) in gemm_roles(cfg).items():
            a = (torch.randn(m, k, generator=gen) * 0.5).to(dev, torch.float16)
            w = (torch.randn(n, k, generator=gen) * k ** -0.5).to(dev, torch.float16)
            bias = torch.randn(n, generator=gen).to(dev)
            bias16 = bias.half()
            out16 = torch.empty(m, n, dtype=torch.float16, device=dev)
            resid = torch.randn(m, n, generator=gen).to(dev) if epi == "resid" else None
            out32 = torch.empty_like(resid) if resid is not None else None
            if epi == "resid":
                ours = lambda: ops.linear_residual(a, w, bias, resid, out=out32)  # noqa: E731
            else:
                ours = lambda: ops.linear(a, w, bias, gelu=epi == "gelu", out=out16)  # noqa: E731
            plain = lambda: ops.linear(a, w, bias, out=out16)  # noqa: E731
            lib = lambda: F.linear(a, w, bias16)  # noqa: E731
            t_lib = timed(lib)
            t_plain = timed(plain)
            t_ours = timed(ours)
            diff = float((plain().float() - lib().float()).abs().max())
            flop = 2.0 * m * n * k
            frac = lambda ms: round(flop / (ms * 1e-3) / (PEAK_FP16_TFLOPS * 1e12), 4)  # noqa: E731
            print(json.dumps({
                "config": name, "role": role, "m": m, "n": n, "k": k, "epilogue": epi,
                "hipblaslt_ms": round(t_lib, 5), "tk_plain_ms": round(t_plain, 5), "tk_ms": round(t_ours, 5),
                "frac_hipblaslt": frac(t_lib), "frac_tk_plain": frac(t_plain), "frac_tk": frac(t_ours),
                "tk_plain_over_hipblaslt": round(t_plain / t_lib, 3),
                "max_abs_diff_plain_vs_hipblaslt": diff,
            }), flush=True)
            del a, w, bias, bias16, out16, resid, out32
            torch.cuda.empty_cache()
    return 0


def layernorm_rotated(configs, reps: int) -> int:
    """Time the library's LayerNorm + cast (tk_ln_cast, fp32 -> fp16, and the
    fp32-out final norm) at each config's [B*S, d_model] on SETS rotated buffer
    sets, so no launch finds its input in the 256 MB Infinity Cache; the mean
    of back-to-back launches between two events.  One JSON line per (config,
    output dtype), with a plain device copy of the same bytes (read fp32,
    write the output dtype) as the achievable reference."""
    from tkmi import ops

    dev = torch.device("cuda:0")
    sets = 4
    for name in configs:
        b, s, d, _, _, _, _ = CONFIGS[name]
        rows = b * s
        w = torch.ones(d, device=dev)
        bias = torch.zeros(d, device=dev)
        xs = [torch.randn(rows, d, device=dev) for _ in range(sets)]
        for out_dtype, per_el in ((torch.float16, 6), (torch.float32, 8)):
            outs = [torch.empty(rows, d, dtype=out_dtype, device=dev) for _ in range(sets)]

            def timed(fn):
                # back-to-back launches between two events: no per-launch event overhead
                for i in range(2 * sets):
                    fn(i % sets)
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for i in range(reps):
                    fn(i % sets)
                e1.record()
                torch.cuda.synchronize()
                return e0.elapsed_time(e1) / reps

            t_ln = timed(lambda i: ops.ln_fwd(xs[i], w, bias, 1e-5, out_dtype))  # noqa: B023
            t_cp = timed(lambda i: outs[i].copy_(xs[i]))  # noqa: B023
            nbytes = float(per_el * rows * d)
            print(json.dumps({
                "config": name, "rows": rows, "cols": d, "out_dtype": str(out_dtype).replace("torch.", ""),
                "buffer_sets": sets, "bytes_per_launch": nbytes,
                "ln_ms": round(t_ln, 5), "ln_frac_hbm": round(nbytes / (t_ln * 1e-3) / (PEAK_HBM_GBPS * 1e9), 4),
                "copy_ms": round(t_cp, 5), "copy_frac_hbm": round(nbytes / (t_cp * 1e-3) / (PEAK_HBM_GBPS * 1e9), 4),
            }), flush=True)
            del outs
        del xs
        torch.cuda.empty_cache()
    return 0


def parse_shape(text: str) -> tuple:
    """``B,S,D,H,F,L[,causal|noncausal]`` -> (B, S, D, H, F, L, causal)."""
    parts = [t.strip() for t in text.split(",") if t.strip()]
    if len(parts) not in (6, 7):
        raise SystemExit(f"--shape wants B,S,D,H,F,L[,causal|noncausal], got {text!r}")
    nums = tuple(int(t) for t in parts[:6])
    causal = True if len(parts) == 6 else parts[6].lower() in ("causal", "c", "1", "true")
    return nums + (causal,)


# CPU work (fp32 flop) above which the CPU leg is skipped instead of sampled.
CPU_FLOP_CAP = 4e12


def cpu_baseline_leg(model, cfg_t, x_host, out_gpu, label: str, mask_host=None):
    """Time the fp32 CPU oracle on a bounded sample of the workload and check
    the GPU output rows the sample covers.  A padded input (``mask_host`` not
    all-true) is sampled only where the whole forward fits the CPU leg (the
    query-chunked oracle is dense-only).
    Returns (cpu_baseline dict or None, parity dict or None)."""
    from oracle import baseline as ob  # the CPU baseline and its parity check only

    b, s, d, h, f, nl, causal = cfg_t
    cfg = ob.TransformerConfig(b, s, d, h, f, nl, causal)
    base = ob.BaselineTransformer(cfg)
    state = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    base.load_state_dict(state, strict=True)
    base = base.eval()
    cores = cpu_cores()
    torch.set_num_threads(cores)
    pairs = s * (s + 1) / 2 if causal else s * s
    flop_per_sample = nl * (2 * s * (4 * d * d + 2 * d * f) + 4 * d * pairs)
    full = b * h * s * s * 4 <= 2 ** 31 and b * flop_per_sample <= CPU_FLOP_CAP
    xs_full = x_host.float()
    parity = None
    if full:
        fn = None if mask_host is None else (lambda t: base(t, mask_host))  # noqa: E731
        xs, sample_b = xs_full, b
        sample = f"full {label} forward (B{b} S{s}), median of 3 after 1 warmup"
        reps, warm = 3, 1
    elif flop_per_sample <= CPU_FLOP_CAP and (mask_host is None or bool(mask_host.all())):
        xs, sample_b = xs_full[:1], 1
        fn = lambda t: ob.chunked_forward(base, t, q_chunk=2048)  # noqa: E731
        sample = (f"query-chunked fp32 oracle (row-exact to the baseline), sequence 0 of the batch of {b}, "
                  f"time x{b}; median of 3 after 1 warmup")
        reps, warm = 3, 1
    else:
        return None, None
    outs = []
    keep = (lambda t: outs.append(fn(t))) if fn is not None else None
    if full and fn is not None:  # padded: the full forward with its mask
        keep = fn
    ts = ob.time_cpu_forward(base, xs, warmup=warm, repeats=reps, fn=keep)
    cpu_fwd = statistics.median(ts) * (b / sample_b)
    cpu = {
        "value": round(cpu_fwd / nl, 3),
        "unit": "ms",
        "cores": cores,
        "kind": "port",
        "sample": sample,
        "forward_ms": round(cpu_fwd, 2),
    }
    if out_gpu is not None:
        if full:
            with torch.inference_mode():
                ref = base(xs) if mask_host is None else base(xs, mask_host)
            got, rows = out_gpu, "every row"
        else:  # the sampled sequence's output from the timed chunked call
            ref, got, rows = outs[-1], out_gpu[:sample_b], f"sequence 0 of {b} (all {s} rows)"
        r = ob.compare_outputs(ref, got)
        parity = {"passed": r.passed, "max_abs": r.max_abs_error, "failed": r.failed_elements,
                  "elements": r.total_elements, "rows": rows, "input": "the timed input (seed 101234)"}
        print(f"[bench] parity {label}: {'PASS' if r.passed else 'FAIL'} max_abs={r.max_abs_error:.3g}",
              file=sys.stderr, flush=True)
    return cpu, parity


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C4", choices=sorted(CONFIGS))
    ap.add_argument("--shape", default=None,
                    help="B,S,D,H,F,L[,causal|noncausal] instead of --config (causal by default)")
    ap.add_argument("--dtype", default="float32", choices=("float32", "float16", "bfloat16"),
                    help="model and input dtype, as the reference harness's --dtype")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-check", action="store_true", help="skip the parity check of the CPU-baseline leg")
    ap.add_argument("--graph", action="store_true",
                    help="time the whole forward replayed from a HIP graph (tkmi.graphs.GraphedTransformer)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of COPY_BYTES (torch copy_), the reference kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    ap.add_argument("--dispatch", nargs="?", const="default", default=None,
                    help="apply the per-shape settings table (tkmi/configs/dispatch.json, or the path given); "
                         "--graph / --unfused-norm given here win")
    ap.add_argument("--padding-ratio", type=float, default=0.0,
                    help="prefix padding masks as the harness's --padding-ratio draws them "
                         "(src/torch_transformer_benchmark.py:255-271); 0 = dense")
    ap.add_argument("--gemm-yardstick", nargs="?", const="C3,C4,C5", default=None,
                    help="only time this build's GEMMs against hipBLASLt (F.linear) on the GEMM roles of the "
                         "given configs (default C3,C4,C5); one JSON line per role")
    ap.add_argument("--layernorm-rotated", nargs="?", const="C2,C3,C4,C5", default=None,
                    help="only time the LayerNorm + cast kernel on rotated buffers at the given configs' "
                         "[B*S, d_model] (default C2,C3,C4,C5), beside a device copy of the same bytes")
    ap.add_argument("--unfused-norm", action="store_true",
                    help="residual GEMM + standalone LayerNorm instead of the fused GEMM+LN epilogue")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one GPU only: this build has no multi-GPU path "
            "(collectives, sharding and rank code are not part of it); run with --gpus 1",
            file=sys.stderr,
        )
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X)", file=sys.stderr)
        return 2

    if args.copy_calibration:
        return copy_calibration()
    if args.gemm_yardstick:
        names = [c.strip() for c in args.gemm_yardstick.split(",") if c.strip()]
        bad = [c for c in names if c not in CONFIGS]
        if bad:
            raise SystemExit(f"--gemm-yardstick: unknown configs {bad}")
        return gemm_yardstick(names, max(args.steps, 3))
    if args.layernorm_rotated:
        names = [c.strip() for c in args.layernorm_rotated.split(",") if c.strip()]
        bad = [c for c in names if c not in CONFIGS]
        if bad:
            raise SystemExit(f"--layernorm-rotated: unknown configs {bad}")
        return layernorm_rotated(names, max(args.steps, 8))

    import tkmi
    from tkmi import ops

    if args.shape:
        cfg_t = parse_shape(args.shape)
        workload = "shape"
    else:
        cfg_t = CONFIGS[args.config]
        workload = args.config
    b, s, d, h, f, nl, causal = cfg_t
    dtype = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[args.dtype]
    dev = torch.device("cuda:0")
    torch.set_num_threads(cpu_cores())
    torch.set_float32_matmul_precision("highest")

    chosen = None
    if args.dispatch:
        from tkmi import dispatch as tkd

        chosen = tkd.settings_for(tkd.load_table(None if args.dispatch == "default" else args.dispatch), *cfg_t)
        if chosen:
            args.graph = args.graph or chosen["graph"]
            args.unfused_norm = args.unfused_norm or not chosen["fused_norm"]
    settings = tkmi.OptimizerSettings(fused_norm=not args.unfused_norm)
    cls = tkmi.OptimizedTransformer
    if args.graph:
        from tkmi.graphs import GraphedTransformer as cls
    torch.manual_seed(1234)  # the harness's construction order and seed
    model = cls(tkmi.TransformerConfig(*cfg_t), settings).to(device=dev, dtype=dtype).eval()
    timed_model = model
    eager = model
    if args.graph:  # built here, outside inference mode: its parameters are ordinary tensors
        eager = tkmi.OptimizedTransformer(tkmi.TransformerConfig(*cfg_t), settings)
        eager.load_state_dict(model.state_dict())
        eager = eager.to(device=dev, dtype=dtype).eval()

    gen = torch.Generator().manual_seed(1234 + 100000)
    x = torch.randn(b, s, d, generator=gen).to(dtype)
    mask = torch.ones(b, s, dtype=torch.bool)
    if args.padding_ratio > 0:
        # the harness's recipe: per-sequence prefix lengths drawn from the same
        # generator after x, padded positions of x zeroed
        min_valid = max(1, int(round(s * (1.0 - args.padding_ratio))))
        lengths = torch.randint(low=min_valid, high=s + 1, size=(b,), generator=gen)
        mask = torch.arange(s)[None, :] < lengths[:, None]
        x = x.masked_fill(~mask[..., None], 0)
    x_host, mask_host = x, mask
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

        # Per-kernel durations: events around each launch, on the launch stream
        # (the eager forward: a replayed graph records no per-launch events).
        with ops.kernel_timer() as rec:
            for _ in range(args.steps):
                eager(x, mask)
            torch.cuda.synchronize()
        got_gpu = model(x, mask).float().cpu() if not args.no_cpu_baseline and not args.no_check else None
        per = {}
        for name, e0, e1 in rec:
            per.setdefault(name, []).append(e0.elapsed_time(e1))

    fwd_ms = statistics.median(samples)
    kernels = {}
    for name, ts in per.items():
        avg_ms = sum(ts) / len(ts)
        kernels[name] = {
            "avg_ms": round(avg_ms, 5),
            "launches_per_step": len(ts) // args.steps,
            "ms_per_step": round(sum(ts) / args.steps, 5),
            **kernel_roofline(name, cfg_t, avg_ms),
        }
        if kernels[name]["bound"] == "hbm":
            # a launch whose bytes fit the 256 MB Infinity Cache may be served from it
            # (the steps re-run the same buffers), so its GB/s is not an HBM figure
            kernels[name]["cache_resident"] = kernels[name]["algorithmic_per_launch"] <= INFINITY_CACHE_BYTES
    dom_name = max(kernels, key=lambda k: kernels[k]["ms_per_step"])
    dom = kernels[dom_name]
    roofline = {
        "kernel": dom_name,
        "bound": dom["bound"],
        "achieved": dom["achieved"],
        "peak": PEAK_FP16_TFLOPS if dom["bound"] == "mfma" else PEAK_HBM_GBPS,
        "unit": dom["unit"],
        "frac": dom["frac"],
        "frac_mfma": dom.get("frac_mfma"),
        "frac_hbm": dom.get("frac_hbm"),
        "traffic": measured_traffic(workload, dom_name) if args.dtype == "float32" else None,
    }
    if roofline["traffic"] is not None:
        # a process cannot count its own dispatches' bytes; the figure is the
        # committed counter run of this same command
        roofline["traffic_source"] = ("profiles/traffic.json: rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, over "
                                      "this bench command, scaled by a plain-copy calibration (x2.0, x1.0)")

    cpu, parity = None, None
    if not args.no_cpu_baseline:
        cpu, parity = cpu_baseline_leg(model, cfg_t, x_host, out_gpu=None if args.no_check else got_gpu,
                                       label=workload, mask_host=mask_host if args.padding_ratio > 0 else None)

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
        "input_dtype": args.dtype,
        "data": "synthetic (seeded randn input, seeded nn.Linear default init)",
        "config": {
            "workload": f"{workload}: B{b} S{s} D{d} H{h} F{f} L{nl} {'causal' if causal else 'non-causal'}",
            "batch": b, "seq_len": s, "d_model": d, "heads": h, "ffn_dim": f, "layers": nl,
            "causal": causal, "parallelism": "single GPU", "fused_norm": not args.unfused_norm,
            "hip_graph": bool(args.graph), "dispatch": chosen, "padding_ratio": args.padding_ratio,
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
