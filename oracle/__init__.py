"""CPU oracle of the grouped MoE-LoRA path — TEST INFRASTRUCTURE ONLY.

A restatement, in numpy (integer work) and PyTorch float32 (products), of what the reference
thinkube/meepsquared computes on this path; every function cites the reference file:line it
follows.  Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import it, and
only as the checker (or, in the bench, as the timed CPU baseline): the product path in
meepsquared_amd/ never routes through it.

How each function is pinned (checked against something other than itself) is stated in its
docstring and exercised by tests/test_oracle.py.
"""
