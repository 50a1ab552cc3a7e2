"""Build librwkv7_hip.so for gfx950 with hipcc (no cmake, no torch extension).

Usage: ``python rwkv-tl_amd/build_hip.py [--jobs N] [--verbose]``.

Every ``csrc/*.hip`` translation unit is compiled to an object in
``_build/`` and linked into ``rwkv_tl_amd/librwkv7_hip.so``. The library
links against ``libamdhip64.so.7`` and ``libhipblaslt.so.1`` (the large-M
plain GEMMs); the Python loader imports torch first, so at run time those
names bind to the HIP runtime and hipBLASLt torch has already loaded.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
OUT = HERE / "rwkv_tl_amd" / "librwkv7_hip.so"
# diagnostic build with the persistent kernels' stage stamps (RWKV7_TIMELINE;
# bench.py --timeline loads it through RWKV7_HIP_LIB)
BUILD_TL = HERE / "_build_timeline"
OUT_TL = HERE / "rwkv_tl_amd" / "librwkv7_hip_timeline.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # no packed fp32 instructions anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{HERE.parent / 'include'}",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")
    return exe


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass reports the device-only target feature; drop that line
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = False, timeline: bool = False) -> Path:
    """Compile every csrc/*.hip and link the shared library; returns its path.
    timeline: the diagnostic library with stage stamps, librwkv7_hip_timeline.so."""
    build_dir, out = (BUILD_TL, OUT_TL) if timeline else (BUILD, OUT)
    build_dir.mkdir(exist_ok=True)
    cc = hipcc()
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [build_dir / (s.stem + ".o") for s in srcs]
    flags = [*COMMON_FLAGS, "-DRWKV7_TIMELINE"] if timeline else COMMON_FLAGS
    cmds = [[cc, *flags, "-c", str(s), "-o", str(o)] for s, o in zip(srcs, objs)]
    jobs = jobs or min(len(cmds), os.cpu_count() or 4, 16)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = out.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-lhipblaslt", "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--timeline", action="store_true",
                    help="build the diagnostic library with stage stamps (librwkv7_hip_timeline.so)")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose, args.timeline))


if __name__ == "__main__":
    main()
