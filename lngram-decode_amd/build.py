"""Build the gfx950 C-ABI library ``lngram_hip/liblngram_hip.so`` from ``csrc/*.hip``.

    python lngram-decode_amd/build.py            # compile (parallel) and link

hipcc cross-compiles for gfx950 without a GPU.  Every HIP translation unit is built
with packed-FP32 instruction selection disabled (``-packed-fp32-ops``).
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OBJ = ROOT / "_build"
LIB = ROOT / "lngram_hip" / "liblngram_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("LNGRAM_ARCH", "gfx950")
FLAGS = [f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]



def _run(cmd: list) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (res.stderr or "").splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [OBJ / (s.stem + ".o") for s in srcs]
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda so: _run([HIPCC, *FLAGS, "-c", str(so[0]), "-o", str(so[1])]), zip(srcs, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, *FLAGS, "-shared", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
