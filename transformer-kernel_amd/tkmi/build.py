"""Build libtkmi.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python -m tkmi.build            # from transformer-kernel_amd/
    python -c "import __graft_entry__ as g; g.build()"   # from the repo root

Every ``csrc/*.hip`` file is compiled to an object under
``transformer-kernel_amd/_build/`` (in parallel), then linked into
``transformer-kernel_amd/tkmi/libtkmi.so``; ``csrc/gen_attn_epochs.py`` and
``csrc/gen_attn_steps64.py`` first rewrite the generated ``csrc/tk_attn_*.inc``.  The flags target gfx950 only.
``-Xclang -target-feature -Xclang -packed-fp32-ops`` keeps the compiler from
emitting packed-fp32 VALU instructions (the host pass warns that it does not
know the feature; that is harmless).

The compiler's per-kernel resource report (registers, scratch, occupancy,
LDS) is saved to ``_build/resource_usage.json``; the host tests check that
the kernels on the benchmarked paths use no scratch memory (a spilled
accumulator makes a kernel several times slower without changing results).
"""

from __future__ import annotations

import concurrent.futures as cf
import json
import os
import pathlib
import re
import shutil
import subprocess
import sys

PKG_DIR = pathlib.Path(__file__).resolve().parent
ROOT = PKG_DIR.parent                     # transformer-kernel_amd/
REPO = ROOT.parent
CSRC = ROOT / "csrc"
INCLUDE = REPO / "include"
BUILD_DIR = ROOT / "_build"
LIB_PATH = PKG_DIR / "libtkmi.so"
RESOURCE_PATH = BUILD_DIR / "resource_usage.json"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def sources():
    return sorted(CSRC.glob("*.hip"))


_REMARK = re.compile(r"remark: +(Function Name|TotalSGPRs|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|"
                     r"Occupancy \[waves/SIMD\]|LDS Size \[bytes/block\]): (\S+)")
_FIELDS = {"TotalSGPRs": "sgprs", "VGPRs": "vgprs", "AGPRs": "agprs", "ScratchSize [bytes/lane]": "scratch",
           "Occupancy [waves/SIMD]": "occupancy", "LDS Size [bytes/block]": "lds"}


def _resource_usage(stderr: str) -> dict:
    """Per-kernel figures from hipcc's -Rpass-analysis=kernel-resource-usage remarks."""
    usage, cur = {}, None
    for m in _REMARK.finditer(stderr):
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = usage.setdefault(val, {})
        elif cur is not None:
            cur[_FIELDS[key]] = int(val)
    return usage


def _compile(src: pathlib.Path):
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr[-4000:]}")
    return obj, _resource_usage(proc.stderr)


def generate() -> None:
    """Write the generated kernel sources (the attention steady-state asm loops)."""
    import importlib.util

    for name in ("gen_attn_epochs", "gen_attn_steps64"):
        spec = importlib.util.spec_from_file_location(name, CSRC / f"{name}.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.write()


def build(verbose: bool = True, jobs: int = 0) -> pathlib.Path:
    """Compile all kernels and link libtkmi.so; returns the library path."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    generate()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(_compile, srcs))
    objs = [obj for obj, _ in results]
    usage = {}
    for _, u in results:
        usage.update(u)
    RESOURCE_PATH.write_text(json.dumps(usage, indent=1, sort_keys=True))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-4000:]}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)
