"""CPU oracle: restatements of the reference's PyTorch paths.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (kernel-pocs_amd/) imports
this package; only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it, as the checker and as the timed CPU baseline.

Each function restates the reference computation it names (file:line,
relative to the Forge-researchlab/kernel-POCs root) with plain PyTorch on the
CPU.  How each one is pinned (checked independently of its own formula) is in
tests/test_oracle.py:

  swiglu.py         closed form in float64 numpy, autograd vs analytic
                    derivative, the reference test's special values
  rope.py           complex-number rotation in numpy complex128, norm
                    preservation, inverse rotation, one-hot gradient
  cross_entropy.py  float64 brute-force log-softmax, F.cross_entropy,
                    gradient row sums, ignore_index semantics
  lora_mlp.py       fp64 gradcheck, autograd of the plain forward composition
  lora_qkv.py       fp64 gradcheck, autograd of the plain forward composition
"""
