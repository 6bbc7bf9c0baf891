"""CPU oracle for the softmax-weighted embedding readout — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this package, and only as the checker (or, in the bench, as the
timed CPU baseline).  The product (``swvr_amd``) never imports it: its path is
the HIP library, and it fails loudly when that library is missing.

Modules
  reference  eager closed form ``softmax(sS + b) E``, ``logsumexp`` and the MSE
             loss, in fp32 / fp64 on the CPU (swvr/reference.py:5-14,
             swvr/api.py:53-66, tests/test_cpu.py:150-159).
  chunked    restatement of the reference's chunked CPU algorithm, forward
             and analytic backward (swvr/chunked.py:82-151); the CPU baseline.

How each function is pinned (tests/test_oracle.py):
  * reference.softmax_readout_reference: brute-force pure-Python loops and
    the committed golden fixtures (tests/golden/), closed forms (V=1, a
    dominant bias, constant scores), the naive exp/sum formula.
  * reference gradients (torch autograd of the closed form): central finite
    differences in fp64 and the fixtures' independently derived gradients.
  * reference.mse_reference: the fixtures' loss values (pure Python).
  * chunked.forward / chunked.backward: against the eager reference and its
    autograd at fp64 across chunk sizes, masked vocabulary, large logits, tied
    W = E and frozen inputs.
"""
