"""Reference module path cuda_autograd_fns.cuda_flash_attention."""
from cuda_transformer_amd.autograd_fns import CudaFlashAttention  # noqa: F401
