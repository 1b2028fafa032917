"""CPU oracle of the QLoRA kernel set — TEST INFRASTRUCTURE ONLY.

Restatements of the reference's algorithms for this path, on the CPU, each citing the
reference file:line it follows:
  nf4_oracle.c / nf4.py   NF4 dequant with double-quantised absmax (plain C, numpy)
  philox.py               the dropout uniform (Philox4x32-10 + Triton's tl.rand mapping, numpy)
  ops.py                  RMSNorm, RoPE, SwiGLU, LoRA cast/add, CE rows, fused head loss
                          (torch fp32 on the CPU)

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline legs may import this
package, and only as the reference results are compared against (or the timed CPU
baseline); the product package `hackathon_amd` never imports it. Each function is pinned by a test against golden vectors, library
routines or invariants (tests/test_oracle_*.py); see the pin list in each module.
"""
