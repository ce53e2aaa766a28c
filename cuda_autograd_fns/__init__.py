"""Reference import path ``cuda_autograd_fns`` -> cuda_transformer_amd.autograd_fns."""
from cuda_transformer_amd.autograd_fns import (  # noqa: F401
    CudaAddLayerNorm, CudaCausalSelfAttention, CudaFlashAttention, CudaFlashAttentionQKV, CudaGeluLayer,
    CudaEmbedding, CudaLayerNorm, CudaLinearLayer, CudaGeluTanhLayer, CudaMLP, CudaSoftmaxLayer,
)

__all__ = ['CudaCausalSelfAttention', 'CudaFlashAttention', 'CudaGeluLayer', 'CudaLinearLayer',
           'CudaSoftmaxLayer', 'CudaLayerNorm', 'CudaMLP', 'CudaGeluTanhLayer',
           'CudaFlashAttentionQKV', 'CudaAddLayerNorm', 'CudaEmbedding']
