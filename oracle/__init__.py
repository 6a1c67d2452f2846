"""CPU oracle for the Rapid-H3 DiT hot path: numpy restatements of the reference's quantizers,
row-wise GEMM epilogues and INT8 attention numerics.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and only as the checker; the product (rapid-h3_amd/) never does.

Pinning (what fixes each function independently of this restatement) is stated in
tests/test_oracle.py; no function here is left unpinned.
"""
