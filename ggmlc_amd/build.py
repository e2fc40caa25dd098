"""Build libgq.so (HIP, gfx950) in-tree: ``python -m ggmlc_amd.build``.

Every .hip file under csrc/ is compiled by hipcc to an object in
ggmlc_amd/_build/ (parallel), then linked into ggmlc_amd/libgq.so. The benchmark's
measurement aids under bench_csrc/ (the streaming-read probe) are linked into their
own ggmlc_amd/libgqbench.so, outside libgq's ABI.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libgq.so"
BENCH_CSRC = PKG / "bench_csrc"
BENCH_LIB = PKG / "libgqbench.so"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # packed fp32 (v_pk_*_f32) stays off: plain float code only
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.parent.name + "_" + src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr}")
    # the host pass warns that it does not know -packed-fp32-ops; anything else is shown
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in r.stderr.splitlines() if noise not in ln)
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def _link(objs, lib: Path) -> None:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    bench_srcs = sorted(BENCH_CSRC.glob("*.hip"))
    jobs = min(len(srcs) + len(bench_srcs), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs + bench_srcs))
    _link(objs[:len(srcs)], LIB)
    _link(objs[len(srcs):], BENCH_LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources, {BENCH_LIB} from {len(bench_srcs)}")
    return LIB


if __name__ == "__main__":
    build()
