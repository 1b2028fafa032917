"""Write tests/golden/triton_rand.json: uniforms drawn by Triton's own tl.rand.

The reference's dropout mask is `tl.rand(seed, (row*N + col).to(int32)) > p`
(solution/lora.py:41-43). This script runs the installed Triton library (not the reference)
on its CPU interpreter (TRITON_INTERPRET=1) for a few seeds, including seeds above 2**32,
and int32 offsets including negative (wrapped) ones, and records the float32 bits.
Run: python tests/golden/make_triton_rand.py
"""

import json
import os
from pathlib import Path

os.environ["TRITON_INTERPRET"] = "1"

import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402


@triton.jit
def _rand_kernel(off_ptr, out_ptr, seed, N, BLOCK: tl.constexpr):
    i = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    offs = tl.load(off_ptr + i, mask=i < N, other=0)
    tl.store(out_ptr + i, tl.rand(seed, offs), mask=i < N)


def main():
    offsets = list(range(0, 40)) + [1535, 1536, 1537, 2**20 + 7, 2**31 - 1, -1, -2, -(2**31),
                                     -123456789, 987654321]
    cases = []
    for seed in (0, 1, 1234, 4321, 2**31 - 2, 2**32 + 5, 0x1234_5678_9ABC):
        offs = torch.tensor(offsets, dtype=torch.int32)
        out = torch.empty(len(offsets), dtype=torch.float32)
        _rand_kernel[(1,)](offs, out, seed, len(offsets), BLOCK=64)
        cases.append({"seed": seed, "offsets": offsets,
                      "bits": [int(b) for b in out.view(torch.int32).tolist()]})
    path = Path(__file__).with_name("triton_rand.json")
    path.write_text(json.dumps({"generator": f"triton {triton.__version__} tl.rand, interpreter",
                                "cases": cases}, indent=0))
    print(path)


if __name__ == "__main__":
    main()
