"""Reference module path cuda_autograd_fns.cuda_softmax_layer."""
from cuda_transformer_amd.autograd_fns import CudaSoftmaxLayer  # noqa: F401
