"""Build the GPU test-support library tests/support/_build/librecip_check.so (hipcc, gfx950)
from recip_check.hip: an exhaustive device check of the SwiGLU kernels' sigmoid. Test
infrastructure only; the product library does not link it."""

import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build" / "librecip_check.so"


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    hipcc = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Wno-unused-command-line-argument", str(HERE / "recip_check.hip"), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed:\n{' '.join(cmd)}\n{proc.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
