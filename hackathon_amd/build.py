"""Build libqlora_gfx950.so, the gfx950 kernel library, in-tree.

Every `csrc/*.hip` file is compiled by hipcc for gfx950 only (no other targets, no host
fallback) and the objects are linked into `hackathon_amd/libqlora_gfx950.so`, which the
Python façades load through ctypes. Run `python -m hackathon_amd.build` (or call
`build()`); it always recompiles.

Device flags:
  -O3 --offload-arch=gfx950
  -Xclang -target-feature -Xclang -packed-fp32-ops
      keeps the compiler from forming packed fp32 (v_pk_*_f32) instructions; the host pass
      prints a harmless "not a recognized feature" warning for it.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB_NAME = "libqlora_gfx950.so"
LIB_PATH = PKG / LIB_NAME
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-file extra flags. nf4.hip must round the product nf4[code] * scale to fp32 before the
# conversion to the output type (the reference's order); with contraction allowed the
# compiler may fuse multiply and conversion into one v_fma_mix with a single rounding.
FILE_FLAGS = {"nf4.hip": ["-ffp-contract=off"]}


def sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> tuple[Path, str]:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, *FILE_FLAGS.get(src.name, []), "-I", str(CSRC), "-c", str(src),
           "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{proc.stderr}")
    noise = "is not a recognized feature for this target"
    warn = "\n".join(l for l in proc.stderr.splitlines() if noise not in l and l.strip())
    return obj, warn


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link the shared library. Returns its path."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(_compile, srcs))
    for obj, warn in results:
        if warn and verbose:
            print(f"[{obj.stem}] {warn}", file=sys.stderr)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o, _ in results]]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)  # atomic: a concurrent loader never sees a half-written file
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose=True)
    print(path)
