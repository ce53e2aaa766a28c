"""The reference's import path (``cuda_transformer``), served by cuda_transformer_amd.

``from cuda_transformer.ops import flash_attention_fwd`` and ``import cuda_transformer``
(which the reference's tests, benchmarks and gpt/gpt.py use) resolve to the gfx950
operator library.
"""
from cuda_transformer_amd import _C, ops  # noqa: F401

__all__ = ["ops"]
