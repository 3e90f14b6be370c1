"""HIP counterpart of the benchmark's grader (graders/child.py, grade.py, verdict.py):
guarded device buffers, the three-call protocol, the tolerance compare, event timing and
verdict labels.  The checker (an fp64 oracle) is passed in by the caller; nothing here
computes reference values itself."""
