"""CPU oracle for the Tiga CSR message-passing hot path.

TEST INFRASTRUCTURE ONLY: a restatement of the reference's algorithms used to
check the HIP provider (tests/, __graft_entry__.smoke()) and to time the
reference's CPU path (bench.py's cpu_baseline leg).  The product never
imports, links or runs anything in this directory.

  ref.py          numpy fp64 restatement of the path (graph indexing, row
                  partition, sum, online softmax, GAT, dot-product, varlen)
  planner.py      the reference's degree-bucket planner decisions
  eager_torch.py  the reference's eager Torch CPU path (timed CPU baseline)
  cpu_native.c    the reference's native CPU forward loop for the sum reducer
                  (timed CPU baseline), built by oracle/Makefile
  native.py       ctypes binding of cpu_native.c
"""
