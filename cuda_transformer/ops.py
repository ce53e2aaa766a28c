"""Reference import path ``cuda_transformer.ops`` -> cuda_transformer_amd.ops."""
from cuda_transformer_amd.ops import *  # noqa: F401,F403
from cuda_transformer_amd.ops import __all__  # noqa: F401
