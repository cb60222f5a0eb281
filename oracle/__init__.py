"""CPU oracle for the SparseFlow spike-sparse convolution path.

TEST INFRASTRUCTURE ONLY.  Nothing under sparseflow_amd/ imports, calls or
links this package; only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it, as the checker.

Modules
  prescan  numpy restatement of the reference's Stage-1 prescan cascade
           (Kernels/_prescan_common.py:32-189) and of this build's bitmap /
           per-tile channel-list formats.
  conv     dense convolution reference (torch F.conv2d on the CPU, the
           library routine the reference itself falls back to and compares
           against: Ops/sparse_conv2d.py:819-834, Benchmark/ops/conv.py:147).
  lif      multi-step LIF closed form (Ops/sparse_fused_conv_lif.py:283-292).
  linear   sparse Linear / batched matmul references (F.linear / torch.bmm
           on the activity-masked operand), the row bitmap and the group
           metadata (Kernels/linear.py:110-357,460; Kernels/bmm.py:66-195).
  brute    independent pure-Python loop forms of the above for tiny inputs,
           used to pin the vectorised restatements.

Pinning status (see tests/test_oracle.py):
  prescan.*         pinned: brute force, torch.max_pool2d, torch fp16 compare
  conv.*            pinned: brute force, F.conv2d, closed-form binary sums
  lif.*             pinned: closed-form constant-current trajectories
  linear.*          pinned: brute-force loops, prescan.active_elements,
                    permutation and linearity identities
  Parity of the reference's Triton tl.dot (fp16) accumulation itself is not
  reproduced (this build computes in fp32 by design).
"""
