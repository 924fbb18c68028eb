"""Run a table of shapes through the benchmark and record the numbers as JSON.

Counterpart of the reference's src/sweep.py: each case runs in its own
subprocess (an out-of-memory or crashing case cannot take the sweep down),
anything after ``--`` is passed to every case's command, a case's own
``extra_args`` follow it, and the results file has the reference's layout
(schema 1: ``config``, ``generated_at``, ``passthrough_args``,
``environment``, ``cases``; src/sweep.py:329-342).  A case runs
``bench.py --shape ...`` (one JSON line, parsed) -- or ``python -m
tkmi.longseq`` when the table marks it ``"runner": "longseq"``.

    python -m tkmi.sweep                                   # the 14 appendix shapes
    python -m tkmi.sweep --config tkmi/configs/baseline.json --cases 1,2
    python -m tkmi.sweep --cases 1,12 --out graph.json -- --graph
    python -m tkmi.sweep --dry-run

Per case the record holds ``status`` (ok / accuracy_failed / error /
timeout), the GPU forward (``optimized``: median ms, tokens/s, per-layer ms,
the dominant kernel's roofline), the CPU oracle's time where bench.py ran
its CPU leg (``baseline``) with the harness's accuracy verdict on the same
input (``accuracy``), and ``speedup`` = CPU time / GPU time.
"""

from __future__ import annotations

import argparse
import json
import pathlib
import subprocess
import sys
import time
from typing import Dict, List, Optional

PKG = pathlib.Path(__file__).resolve().parent
REPO = PKG.parents[1]
BENCH = REPO / "bench.py"
DEFAULT_TABLE = PKG / "configs" / "shapes.json"


def case_command(case: Dict, passthrough: List[str]) -> List[str]:
    causal = "causal" if case.get("causal", True) else "noncausal"
    if case.get("runner") == "longseq":
        cmd = [sys.executable, "-m", "tkmi.longseq",
               "--batch-size", str(case["batch_size"]), "--seq-len", str(case["seq_len"]),
               "--d-model", str(case["d_model"]), "--heads", str(case["heads"]),
               "--ffn-dim", str(case["ffn_dim"]), "--layers", str(case["layers"])]
        if causal == "noncausal":
            cmd.append("--non-causal")
        return cmd + list(case.get("extra_args", []))
    shape = ",".join(str(case[k]) for k in ("batch_size", "seq_len", "d_model", "heads", "ffn_dim", "layers"))
    return [sys.executable, str(BENCH), "--shape", f"{shape},{causal}"] + passthrough + list(case.get("extra_args", []))


def _last_json(stdout: str) -> Optional[Dict]:
    for line in reversed(stdout.strip().splitlines()):
        line = line.strip()
        if line.startswith("{"):
            try:
                return json.loads(line)
            except ValueError:
                return None
    return None


def parse_result(case: Dict, line: Optional[Dict]) -> Dict:
    """The record fields the reference's results carry, from one JSON line."""
    if line is None:
        return {}
    if case.get("runner") == "longseq":
        return {"optimized": {"median_ms": line.get("ms_median"), "tokens_per_second": line.get("tokens_per_s"),
                              "layer_ms": line.get("layer_ms"), "mode": line.get("mode")}}
    out = {
        "optimized": {"median_ms": line.get("ms_per_step"), "tokens_per_second": line.get("tokens_per_s"),
                      "layer_ms": line.get("value"), "roofline": line.get("roofline")},
        "dtype": line.get("input_dtype"),
        "gpu": line.get("device"),
    }
    cpu = line.get("cpu_baseline")
    if cpu:
        out["baseline"] = {"median_ms": cpu.get("forward_ms"), "kind": "fp32 CPU oracle", "cores": cpu.get("cores"),
                           "sample": cpu.get("sample")}
        if line.get("ms_per_step"):
            out["speedup"] = cpu["forward_ms"] / line["ms_per_step"]
    par = line.get("parity")
    if par:
        out["accuracy"] = {"passed": par["passed"], "max_abs_error": par["max_abs"],
                           "failed_elements": par["failed"], "total_elements": par["elements"]}
    return out


def classify(returncode: int, parsed: Dict, timed_out: bool) -> str:
    if timed_out:
        return "timeout"
    if returncode != 0 or "optimized" not in parsed:
        return "error"
    if parsed.get("accuracy") and not parsed["accuracy"]["passed"]:
        return "accuracy_failed"
    return "ok"


def run_case(case: Dict, passthrough: List[str], timeout: float, verbose: bool) -> Dict:
    command = case_command(case, passthrough)
    started = time.time()
    timed_out = False
    cwd = str(PKG.parent) if case.get("runner") == "longseq" else str(REPO)
    try:
        done = subprocess.run(command, capture_output=True, text=True, timeout=timeout, cwd=cwd)
        stdout, stderr, rc = done.stdout, done.stderr, done.returncode
    except subprocess.TimeoutExpired as exc:
        timed_out = True
        stdout = exc.stdout.decode(errors="replace") if isinstance(exc.stdout, bytes) else (exc.stdout or "")
        stderr = exc.stderr.decode(errors="replace") if isinstance(exc.stderr, bytes) else (exc.stderr or "")
        rc = -1
    if verbose:
        print(stdout, end="")
        print(stderr, end="", file=sys.stderr)
    parsed = parse_result(case, _last_json(stdout))
    record = {"case": case, "command": command, "status": classify(rc, parsed, timed_out), "returncode": rc,
              "wall_seconds": round(time.time() - started, 2), **parsed}
    if record["status"] != "ok":
        record["stderr_tail"] = "\n".join(stderr.strip().splitlines()[-12:])
    return record


def _fmt(v, spec=".3f", suffix=""):
    return "-" if v is None else f"{v:{spec}}{suffix}"


def format_table(records: List[Dict]) -> str:
    head = f"{'#':>3}  {'shape':<34} {'status':<16} {'gpu ms':>10} {'cpu ms':>10} {'speedup':>9}  {'max_abs':>9}"
    lines = [head, "-" * len(head)]
    for r in records:
        c = r["case"]
        shape = f"b{c['batch_size']} s{c['seq_len']} d{c['d_model']} h{c['heads']} l{c['layers']} f{c['ffn_dim']}"
        opt, base, acc = r.get("optimized") or {}, r.get("baseline") or {}, r.get("accuracy") or {}
        lines.append(f"{c['id']:>3}  {shape:<34} {r['status']:<16} {_fmt(opt.get('median_ms')):>10} "
                     f"{_fmt(base.get('median_ms')):>10} {_fmt(r.get('speedup'), '.1f', 'x'):>9}  "
                     f"{_fmt(acc.get('max_abs_error'), '.2e'):>9}")
    return "\n".join(lines)


def main(argv: Optional[List[str]] = None) -> int:
    argv = list(sys.argv[1:] if argv is None else argv)
    passthrough: List[str] = []
    if "--" in argv:
        i = argv.index("--")
        argv, passthrough = argv[:i], argv[i + 1:]
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--config", default=str(DEFAULT_TABLE), help="JSON table with a 'cases' list")
    ap.add_argument("--cases", default="", help="comma-separated case ids to run (default: all)")
    ap.add_argument("--skip", default="", help="comma-separated case ids to skip")
    ap.add_argument("--out", default=None, help="results path (default: results/<table>-<time>.json)")
    ap.add_argument("--timeout", type=float, default=900.0)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--dry-run", action="store_true", help="print the commands and exit")
    args = ap.parse_args(argv)

    table = json.loads(pathlib.Path(args.config).read_text())
    cases = table["cases"]
    if args.cases:
        want = {int(v) for v in args.cases.split(",") if v.strip()}
        cases = [c for c in cases if c["id"] in want]
    if args.skip:
        drop = {int(v) for v in args.skip.split(",") if v.strip()}
        cases = [c for c in cases if c["id"] not in drop]
    if not cases:
        print("no cases selected", file=sys.stderr)
        return 1
    if args.dry_run:
        for c in cases:
            print(" ".join(case_command(c, passthrough)))
        return 0

    records = []
    for n, case in enumerate(cases, start=1):
        print(f"[{n}/{len(cases)}] case {case['id']} ...", flush=True)
        rec = run_case(case, passthrough, args.timeout, args.verbose)
        records.append(rec)
        opt = rec.get("optimized") or {}
        print(f"    {rec['status']} | gpu {_fmt(opt.get('median_ms'))} ms", flush=True)

    first = next((r for r in records if r.get("gpu")), None)
    payload = {
        "schema": 1,
        "config": table.get("name", pathlib.Path(args.config).stem),
        "generated_at": time.strftime("%Y-%m-%dT%H:%M:%S%z"),
        "passthrough_args": passthrough,
        "environment": {"gpu": first.get("gpu") if first else None,
                        "torch": __import__("torch").__version__,
                        "dtype": first.get("dtype") if first else None},
        "cases": records,
    }
    out = pathlib.Path(args.out or REPO / "results" / f"{payload['config']}-{time.strftime('%Y%m%d-%H%M%S')}.json")
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(payload, indent=2) + "\n")
    print()
    print(format_table(records))
    print(f"\nwrote {out}")
    return 0 if all(r["status"] == "ok" for r in records) else 1


if __name__ == "__main__":
    sys.exit(main())
