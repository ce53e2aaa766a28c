"""Reference module path cuda_autograd_fns.cuda_causal_self_attention."""
from cuda_transformer_amd.autograd_fns import CudaCausalSelfAttention  # noqa: F401
