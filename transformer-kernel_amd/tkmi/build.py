"""Build libtkmi.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python -m tkmi.build            # from transformer-kernel_amd/
    python -c "import __graft_entry__ as g; g.build()"   # from the repo root

Every ``csrc/*.hip`` file is compiled to an object under
``transformer-kernel_amd/_build/`` (in parallel), then linked into
``transformer-kernel_amd/tkmi/libtkmi.so``.  The flags target gfx950 only.
``-Xclang -target-feature -Xclang -packed-fp32-ops`` keeps the compiler from
emitting packed-fp32 VALU instructions (the host pass warns that it does not
know the feature; that is harmless).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
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


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr[-4000:]}")
    return obj


def build(verbose: bool = True, jobs: int = 0) -> pathlib.Path:
    """Compile all kernels and link libtkmi.so; returns the library path."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, srcs))
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
