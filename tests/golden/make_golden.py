#!/usr/bin/env python3
"""Write golden vectors from the reference implementation (run in the build container only).

The reference's model, input generator and accuracy rule are Python on torch.
Closed forms and the float64 twin pin the oracle's arithmetic to tolerance,
but only the reference itself pins two things bit-exactly:

  * the seeded weights (RNG consumption order of the module construction), and
  * the exact fp32 CPU output of ``BaselineTransformer`` on seeded inputs.

This script imports ``src/torch_transformer_benchmark.py`` from the reference
checkout (path given by --reference, default /root/reference), evaluates it on
small configurations and stores inputs/outputs and hashes as data in
``tests/golden/golden.npz`` and ``tests/golden/golden.json``.  Nothing from the
reference is copied; the fixtures are numbers only.  The GPU box never runs
this script (the reference is absent there).

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import argparse
import hashlib
import json
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent

# Small configs whose full inputs/outputs are stored.
SMALL = {
    "tiny_causal": dict(batch_size=2, seq_len=16, d_model=64, num_heads=4, ffn_dim=128, num_layers=2, causal=True),
    "tiny_full": dict(batch_size=2, seq_len=8, d_model=32, num_heads=2, ffn_dim=48, num_layers=1, causal=False),
    "c1_b1": dict(batch_size=1, seq_len=128, d_model=128, num_heads=4, ffn_dim=128, num_layers=4, causal=True),
    "c2_s16": dict(batch_size=1, seq_len=16, d_model=512, num_heads=8, ffn_dim=2048, num_layers=4, causal=False),
}
# Padded-mask case (future padding path): output stored too.
PADDED = ("tiny_padded", dict(batch_size=3, seq_len=16, d_model=64, num_heads=4, ffn_dim=128, num_layers=1, causal=True), 0.3)

# The five benchmark configs: only hashes of weights and inputs are stored.
FULL = {
    "C1": dict(batch_size=64, seq_len=128, d_model=128, num_heads=4, ffn_dim=128, num_layers=4, causal=True),
    "C2": dict(batch_size=256, seq_len=64, d_model=512, num_heads=8, ffn_dim=2048, num_layers=4, causal=False),
    "C3": dict(batch_size=8, seq_len=2048, d_model=1024, num_heads=16, ffn_dim=4096, num_layers=6, causal=True),
    "C4": dict(batch_size=4, seq_len=8192, d_model=2048, num_heads=16, ffn_dim=8192, num_layers=2, causal=True),
    "C5": dict(batch_size=2, seq_len=32768, d_model=1024, num_heads=16, ffn_dim=4096, num_layers=1, causal=True),
}

SEED = 1234


def state_hash(module) -> str:
    h = hashlib.sha256()
    for key, value in module.state_dict().items():
        h.update(key.encode())
        h.update(value.detach().contiguous().cpu().numpy().tobytes())
    return h.hexdigest()


def tensor_hash(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().contiguous().cpu().numpy().tobytes()).hexdigest()


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--skip-full", action="store_true")
    args = ap.parse_args()
    sys.path.insert(0, str(pathlib.Path(args.reference) / "src"))
    import torch_transformer_benchmark as ref  # noqa: E402  (reference, this container only)

    torch.set_num_threads(8)
    torch.set_float32_matmul_precision("highest")
    arrays = {}
    meta = {"seed": SEED, "torch": torch.__version__, "small": {}, "full": {}}

    def run_small(name, cfg_kw, padding):
        cfg = ref.TransformerConfig(**cfg_kw)
        torch.manual_seed(SEED)
        model = ref.BaselineTransformer(cfg).eval()
        x, mask = ref.generate_random_case(cfg, torch.device("cpu"), torch.float32, SEED, padding, 1.0)
        with torch.inference_mode():
            out = model(x, mask)
        arrays[f"{name}.x"] = x.numpy()
        arrays[f"{name}.mask"] = mask.numpy()
        arrays[f"{name}.out"] = out.numpy()
        meta["small"][name] = {"config": cfg_kw, "padding_ratio": padding, "state_sha256": state_hash(model)}

    for name, kw in SMALL.items():
        run_small(name, kw, 0.0)
    run_small(PADDED[0], PADDED[1], PADDED[2])

    # compare_outputs on hand-built vectors covering every branch of the rule.
    ref_v = torch.tensor([1.0, 0.05, 0.05, -2.0, 0.0, 1.0, float("nan"), 3.0, 1e-4])
    opt_v = torch.tensor([1.019, 0.0519, 0.0521, -2.05, 0.002, float("inf"), 1.0, 3.0, 0.0021])
    res = ref.compare_outputs(ref_v, opt_v, rtol=0.02, atol=0.002)
    arrays["cmp.ref"] = ref_v.numpy()
    arrays["cmp.opt"] = opt_v.numpy()
    meta["compare_outputs"] = {
        "passed": res.passed,
        "failed_elements": res.failed_elements,
        "failed_feature_dims": res.failed_feature_dims,
    }

    if not args.skip_full:
        for name, kw in FULL.items():
            cfg = ref.TransformerConfig(**kw)
            torch.manual_seed(SEED)
            model = ref.BaselineTransformer(cfg)
            x, _ = ref.generate_random_case(cfg, torch.device("cpu"), torch.float32, SEED, 0.0, 1.0)
            meta["full"][name] = {"config": kw, "state_sha256": state_hash(model), "x_sha256": tensor_hash(x)}
            del model, x
            print(name, "hashed", flush=True)

    np.savez_compressed(HERE / "golden.npz", **arrays)
    (HERE / "golden.json").write_text(json.dumps(meta, indent=1) + "\n")
    print("wrote", HERE / "golden.npz", HERE / "golden.json")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
