"""Reference module path cuda_autograd_fns.cuda_linear_layer."""
from cuda_transformer_amd.autograd_fns import CudaLinearLayer  # noqa: F401
