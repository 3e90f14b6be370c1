"""Grading the drop-in kernels on device memory.

- signature: a task's C++ entry as parameters, and the `grader_entry(void**)` shim text;
- entry: calling a drop-in library through that shim;
- arena: one guarded allocation per case (4 KiB 0xA5 gaps, 0xFF-filled outputs) and the
  check that nothing outside the outputs moved;
- protocol: the three calls of a case (set A, set B at the same addresses, set A again),
  and timing a case;
- tolerance: per-element agreement with the oracle;
- labels: failure labels and the pass / fail / flip status over passes;
- clock: hipEvent ms per call;
- ledger: verdict rows and tables from grading logs.

The expected values come from a checker the caller passes in (the tests pass the oracle);
nothing here computes reference values itself."""
