"""CPU oracle for the Mamba-3 chunked-SSD forward path — TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s cpu_baseline leg may import
this package, and only as the checker / the timed CPU baseline. The product
(`mamba3_amd`) never imports it and has no CPU fallback.

Modules
-------
reference_path
    PyTorch-CPU restatement of the reference's algorithm (factored-cumsum intra-chunk
    output, torch-loop chunk scan, op-for-op decode step), each function citing the
    reference file:line it follows. Pinned by: the golden vectors written from the
    reference (tests/golden), the fp64 recurrence below, and closed forms (see
    tests/test_oracle.py).
recurrence
    Float64 token-by-token recurrence (the decode-step equations), plus a brute-force
    L-matrix evaluation of the scalar-decay SSD, used as ground truth.
"""
