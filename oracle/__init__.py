"""Oracle: CPU restatements of the reference's chunk-32 GEMM
(f16acc/kernel.py:37-105 of the reference).

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import, call, link or execute anything here,
and only as the checker (or the reported CPU baseline), never as the thing
measured or shipped.  The product path (f16acc_amd) never imports it.

chunk32.py   PyTorch-CPU restatement (fast; batched FP32 products per chunk)
chunk32.c    scalar C restatement (fixed sequential order), via c_oracle.py

Parity pinning of each function is done by tests/test_oracle.py: closed forms
from the reference's own tests (tests/test_f16acc.py:91-101 of the reference),
constructed inputs whose chunked / FP32 / per-tile-redo results differ in
closed form, exhaustive FP16 conversion against numpy, brute force against
the scalar C code, and the reference's published FP64 error levels
(tests/test_f16acc.py:39-40, README.md:29 of the reference).
"""
