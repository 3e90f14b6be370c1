"""CPU oracle for the six task ops — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker (or, for the CPU baseline, as the timed CPU path).  The
product path (libtaskops.so and the cob_amd package) never imports or calls it.

Modules:
  exact  — numpy fp64 restatements of each task's `reference_exact` (the correctness
           reference; leaky's is the fp32 step loop, fp8_linear's rounds once to bf16).
  eager  — fp32 PyTorch-CPU restatements of each task's eager `reference` (the reported
           CPU baseline), following the reference's op sequence.
  e4m3   — the OCP E4M3 decode table built from the format definition.

Every function cites the reference file:line it follows.  How each one is pinned
(golden input digests, closed forms, invariants, brute force) is in tests/test_oracle.py;
no function here is "parity unpinned".
"""
