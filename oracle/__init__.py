"""CPU oracle for the SimSD matmul hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only to check results against it (or, for the CPU baseline,
as the timed CPU path).  The product path in simsd-release_amd/ never calls it.

  oracle.numerics     bf16/fp16 rounding (numpy, and pure-integer for fixtures)
  oracle.thin_linear  the skinny linear: exact-sum reference + torch-CPU F.linear
  oracle.moe          routing top-k, align tables, per-expert MoE loop
"""
