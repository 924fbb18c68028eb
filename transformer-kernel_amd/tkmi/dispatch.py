"""Per-shape settings dispatch generated from measured sweeps.

Counterpart of the reference's src/dispatch.py: scan sweep results
(``python -m tkmi.sweep`` files, schema 1), keep the fastest accuracy-passing
run per shape, and write the winning settings to a table that
``bench.py --dispatch`` (or ``settings_for``) applies to a shape.

The settings this build can vary per shape are the Python-level ones:
``graph`` (replay the forward from a HIP graph, tkmi.graphs) and
``fused_norm`` (GEMM+LayerNorm epilogue vs residual GEMM + LayerNorm).
Tile and wave-count choices are made per shape inside the kernels' own C
dispatch and are not part of the table.

    python -m tkmi.dispatch results/*.json                 # -> tkmi/configs/dispatch.json
    python -m tkmi.dispatch a.json b.json --out table.json

Rules (src/dispatch.py:24-37): only status-ok records compete; settings
given explicitly on the command line beat the table; medians from
different sweep files come from different sessions, so near-ties are ties
-- the table keeps each winner's source file for re-measurement.
"""

from __future__ import annotations

import argparse
import json
import pathlib
import sys
import time
from typing import Dict, Iterable, Optional

PKG = pathlib.Path(__file__).resolve().parent
DEFAULT_TABLE = PKG / "configs" / "dispatch.json"
SHAPE_FIELDS = ("batch_size", "seq_len", "d_model", "heads", "ffn_dim", "layers", "causal")


def shape_key(case: Dict) -> str:
    return ",".join(str(case[k]) for k in SHAPE_FIELDS)


def settings_of(passthrough: Iterable[str], extra: Iterable[str]) -> Dict[str, bool]:
    args = list(passthrough) + list(extra)
    return {"graph": "--graph" in args, "fused_norm": "--unfused-norm" not in args}


def build_table(paths: Iterable[pathlib.Path]) -> Dict:
    best: Dict[str, Dict] = {}
    sources = []
    for path in paths:
        data = json.loads(pathlib.Path(path).read_text())
        if data.get("schema") != 1:
            continue
        sources.append(pathlib.Path(path).name)
        for rec in data.get("cases", []):
            opt = rec.get("optimized") or {}
            ms = opt.get("median_ms")
            if rec.get("status") != "ok" or ms is None or rec["case"].get("runner"):
                continue
            key = shape_key(rec["case"])
            if key not in best or ms < best[key]["median_ms"]:
                best[key] = {"shape": {k: rec["case"][k] for k in SHAPE_FIELDS},
                             "settings": settings_of(data.get("passthrough_args", []),
                                                     rec["case"].get("extra_args", [])),
                             "median_ms": ms, "source": pathlib.Path(path).name}
    return {"schema": 1, "generated_at": time.strftime("%Y-%m-%dT%H:%M:%S%z"), "sources": sources,
            "shapes": sorted(best.values(), key=lambda e: shape_key(e["shape"]))}


def load_table(path: Optional[pathlib.Path] = None) -> Dict:
    return json.loads(pathlib.Path(path or DEFAULT_TABLE).read_text())


def settings_for(table: Dict, batch_size: int, seq_len: int, d_model: int, heads: int, ffn_dim: int,
                 layers: int, causal: bool) -> Optional[Dict[str, bool]]:
    """The table's settings for this shape, or None when it has no entry."""
    key = ",".join(str(v) for v in (batch_size, seq_len, d_model, heads, ffn_dim, layers, causal))
    for entry in table.get("shapes", []):
        if shape_key(entry["shape"]) == key:
            return dict(entry["settings"])
    return None


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("results", nargs="+", help="sweep results files (schema 1)")
    ap.add_argument("--out", default=str(DEFAULT_TABLE))
    args = ap.parse_args(argv)
    table = build_table(pathlib.Path(p) for p in args.results)
    pathlib.Path(args.out).write_text(json.dumps(table, indent=2) + "\n")
    print(f"wrote {args.out}: {len(table['shapes'])} shapes from {len(table['sources'])} files")
    return 0


if __name__ == "__main__":
    sys.exit(main())
