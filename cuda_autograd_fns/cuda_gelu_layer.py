"""Reference module path cuda_autograd_fns.cuda_gelu_layer."""
from cuda_transformer_amd.autograd_fns import CudaGeluLayer  # noqa: F401
