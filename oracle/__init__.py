"""CPU oracle for sid's decode hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in plain fp32 torch on the CPU (integer work in numpy/int64),
the algorithm of each op on the path, citing the reference file:line each function
follows (paths relative to the sid repository). It is the checker: only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import it. The product
(deterministic-inference_amd/) never imports it and has no CPU fallback.

Pinning (what checks each function beyond itself) is listed per module; see
tests/test_oracle.py for the checks.
"""
