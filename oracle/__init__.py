"""CPU oracle for clustered sparse decode attention: TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import, call or link
anything here, and only as the checker (or, in bench.py, as the timed CPU baseline). The
product (the ssa_amd package and libssa_hip.so) never uses it.

  canon.c / canon.py   the cluster index (prefill fit, insertion + split, selection, compaction)
                       restated in the canonical fp32 order of operations: compared bit for bit
  reference.py         numpy float64 restatement of the reference's PyTorch functions (attention
                       spec, merge, stable rank mask, bisection, k-means, byte accounting)

Every function cites the reference file:line it follows. How each is pinned (golden vectors,
closed forms, invariants, brute force) is listed in tests/test_oracle.py; the reference
repository holds no golden tensors for this path.
"""
