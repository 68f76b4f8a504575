"""CPU oracle for the fused dequant + GEMV path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference's algorithm for the decode
path of KrishnaI2424/Dequant_Project:

  packer_ref.py   numpy restatement of dequant/packer.py (quantize, pack,
                  unpack, dequantize) plus the tests' exact_weight and the
                  fp32-accumulation criterion (scripts/test_dequant_kernel.py).
  cpu_path.py     torch-CPU restatement of the reference's CPU torch path
                  (unpack -> dequantize -> F.linear), timed as the CPU
                  baseline by bench.py.
  dq_oracle.c     scalar C restatement of unpack / dequantize / the GEMV
                  reference, built by oracle/Makefile into
                  oracle/_build/libdq_oracle.so.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this package, and only as the checker (or, for cpu_path, as the timed CPU
baseline). The product path (dequant_project_amd) never imports it and has no
CPU fallback.

Parity status of each function is recorded in the module docstrings; every
function here is pinned by known-answer vectors or closed-form checks under
tests/ (see tests/test_oracle.py).
"""
