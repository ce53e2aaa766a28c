"""CPU oracle for the FP32 transformer kernel set — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's algorithms (CUDA_Transformer, file:line cited on
every function), used as the checker of the HIP kernels.  It is never part of the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import it, and only to check or to time the CPU path.  The operators in
``cuda_transformer_amd`` never call into it.

Pinning (tests/test_oracle.py, all CPU):
  * attention.fa2_forward / fa2_backward — against torch's SDPA math path + autograd in
    float64 (the reference's own test oracle, test/test_flash_attention.py:10-50), the committed
    golden fixtures, closed forms (causal row 0, K = 0, constant V, T = 1), invariants
    (sum_j dK_j = 0, sum_j dV_j = sum_i dO_i) and central finite differences.
  * linear — numpy matmul in float64, identity/one-hot closed forms, finite differences;
    linear.mlp_forward / mlp_backward (fc1 -> GELU -> fc2) against torch float64 autograd and a
    finite difference through both layers.
  * gelu — erf closed form at known points, finite differences for the gradient.
  * gelu_tanh — torch's float64 F.gelu(approximate="tanh") + autograd, the identity
    y(x) - y(-x) = x, its distance to the erf GELU, finite differences.
  * softmax — row sums, shift invariance, torch autograd, finite differences.
  * layernorm — torch.nn.functional.layer_norm + autograd, normalisation invariants.
  * naive attention — torch math of test/test_causal_self_attn.py:10-30 + autograd.
Mutation tests plant plausible mistakes (wrong scale, dropped mask, transposed operand, missing
delta term, a dropped or mis-differentiated tanh-GELU term) in copies of the oracle and check that these checks catch them.
"""
from . import attention, elementwise, linear  # noqa: F401

__all__ = ["attention", "elementwise", "linear"]
