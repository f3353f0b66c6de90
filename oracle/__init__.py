"""Oracle: CPU restatement of the reference's hot-path arithmetic.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this package, and only as the checker
(or, in bench.py, as the timed CPU baseline).  The product path
(braidinfer_amd/) never imports, calls or falls back to anything here.

Two independent restatements:
  oracle.torch_ref  the reference's own torch op sequences on CPU tensors,
                    same calls and the same rounding points (file:line cited
                    per function); the Triton-only fused kernels are restated
                    at their rounding points.
  oracle.numpy_ref  the same mathematics in numpy float64 with bf16/fp16
                    rounding emulated bit-exactly at the same points; used to
                    pin oracle.torch_ref (a dropped term, wrong sign, wrong
                    index or transposed operand in either shows up as a
                    disagreement).
Every function is pinned by tests/test_oracle.py and tests/test_golden.py
(closed forms, invariants, the reference tests' own checks and fixtures, brute
force on tiny inputs, and the numpy-vs-torch cross check).  No function is
parity unpinned.
"""
