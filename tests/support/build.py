"""Build the GPU test-support libraries (hipcc, gfx950) into tests/support/_build/:

  librecip_check.so    recip_check.hip: an exhaustive device check of the SwiGLU kernels'
                       sigmoid
  libqlora_dmacheck.so the attention kernels (hackathon_amd/csrc/attention.hip, with api.hip)
                       built with -DQL_DMA_CHECK: the direct-to-LDS ordering check counts
                       violations in a device counter (qlora_debug_dma_violations)

Test infrastructure only; the product library links neither."""

import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build" / "librecip_check.so"
DMA_CHECK = HERE / "_build" / "libqlora_dmacheck.so"
CSRC = HERE.parent.parent / "hackathon_amd" / "csrc"


def _hipcc(out: Path, sources, defines=()) -> Path:
    out.parent.mkdir(exist_ok=True)
    hipcc = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Wno-unused-command-line-argument", "-I", str(CSRC), *defines,
           *[str(x) for x in sources], "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed:\n{' '.join(cmd)}\n{proc.stderr}")
    os.replace(tmp, out)
    return out


def build() -> Path:
    _hipcc(OUT, [HERE / "recip_check.hip"])
    _hipcc(DMA_CHECK, [CSRC / "attention.hip", CSRC / "api.hip"], ["-DQL_DMA_CHECK"])
    return OUT.parent


if __name__ == "__main__":
    print(build())
