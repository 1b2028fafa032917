"""Build the C oracle (oracle/nf4_oracle.c) into oracle/_build/liboracle.so with gcc.

Test infrastructure only. -ffp-contract=off keeps every fp32 multiply and add separately
rounded, as the restated reference formula requires.
"""

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build" / "liboracle.so"


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared",
           str(HERE / "nf4_oracle.c"), "-o", str(tmp)]
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
