"""ctypes binding of the C ABI in ``include/cuda_transformer_amd.h``.

This is the binding a non-torch caller would use; other FFIs (cgo, JNI, N-API) bind the same
symbols.  The tests use it to call the kernels through the C boundary directly and to check
that the shared library exports every declared symbol.  Loading it needs no GPU.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libcuda_transformer_amd.so"
HEADER = _PKG.parent / "include" / "cuda_transformer_amd.h"

_i64 = ctypes.c_int64
_p = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)
_int = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes)
SIGNATURES = {
    "cta_last_error": (ctypes.c_char_p, []),
    "cta_version": (ctypes.c_char_p, []),
    "cta_flash_attention_fwd": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _i64, _i64, _i64, _i64,
                                       _int, _p, _p, _p]),
    "cta_flash_attention_fwd_bf16": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _i64, _i64, _i64,
                                            _i64, _int, _p, _p, _p]),
    "cta_flash_attention_bwd_workspace": (_i64, [_i64, _i64, _i64, _i64, _int]),
    "cta_flash_attention_bwd_split_workspace": (_i64, [_i64, _i64, _i64, _i64, _int]),
    "cta_flash_attention_bwd": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p,
                                       _p, _i64p, _i64, _i64, _i64, _i64, _int, _p, _p, _p, _p,
                                       _p, _i64, _p]),
    "cta_flash_attention_fwd_strided": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _i64, _i64, _i64,
                                               _i64, _int, _p, _i64p, _p, _p]),
    "cta_flash_attention_fwd_workspace": (_i64, [_i64, _i64, _i64, _i64, _int]),
    "cta_flash_attention_fwd_ex": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _i64, _i64, _i64, _i64,
                                          _int, _p, _i64p, _p, _p, _i64, _p]),
    "cta_flash_attention_bwd_strided": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p,
                                               _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _int,
                                               _p, _i64p, _p, _i64p, _p, _i64p, _p, _p, _i64,
                                               _p]),
    "cta_flash_attention_bwd_noalloc": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p,
                                               _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _int,
                                               _p, _p, _p, _p]),
    "cta_flash_attention_fwd_f16": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _i64, _i64, _i64,
                                           _i64, _int, _p, _p, _p]),
    "cta_flash_attention_bwd_f16_workspace": (_i64, [_i64, _i64, _i64, _i64, _int]),
    "cta_flash_attention_bwd_f16": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p,
                                           _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _int, _p,
                                           _p, _p, _p, _p, _i64, _p]),
    "cta_flash_attention_bwd_bf16_workspace": (_i64, [_i64, _i64, _i64, _i64, _int]),
    "cta_flash_attention_bwd_bf16": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p,
                                            _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _int, _p,
                                            _p, _p, _p, _p, _i64, _p]),
    "cta_flash_attention_bwd_delta": (_int, [_p, _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _p,
                                             _p]),
    "cta_flash_attention_bwd_dq": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p,
                                          _p, _i64, _i64, _i64, _i64, _int, _p, _p]),
    "cta_flash_attention_bwd_dq_delta": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p,
                                                _i64p, _p, _i64p, _i64, _i64, _i64, _i64, _int,
                                                _p, _p, _p]),
    "cta_flash_attention_bwd_dkdv": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p,
                                            _i64p, _p, _i64, _i64, _i64, _i64, _int, _p, _p,
                                            _p]),
    "cta_flash_attention_bwd_dkdv_store_ds": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _p,
                                                     _i64p, _p, _i64p, _p, _i64, _i64, _i64,
                                                     _i64, _int, _p, _p, _p, _p]),
    "cta_flash_attention_bwd_dq_from_ds": (_int, [_p, _i64p, _p, _i64, _i64, _i64, _i64, _int,
                                                  _p, _p]),
    "cta_flash_attention_bwd_fold_delta": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p,
                                                  _p, _i64p, _p, _i64p, _i64, _i64, _i64, _i64,
                                                  _int, _p, _p, _p, _p, _i64, _p]),
    "cta_cuda_fma_workspace": (_i64, [_i64, _i64, _i64, _i64]),
    "cta_cuda_fma": (_int, [_p, _i64p, _p, _i64p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p,
                            _p, _p]),
    "cta_cuda_fma_gelu": (_int, [_p, _i64p, _p, _i64p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _p, _p, _p, _p]),
    "cta_cuda_fma_gelu_grad": (_int, [_p, _i64p, _p, _i64p, _p, _i64, _i64, _i64, _i64, _i64,
                                      _p, _p, _p]),
    "cta_cuda_fma_gelu_tanh": (_int, [_p, _i64p, _p, _i64p, _p, _i64, _i64, _i64, _i64, _i64,
                                      _i64, _p, _p, _p, _p]),
    "cta_cuda_fma_gelu_tanh_grad": (_int, [_p, _i64p, _p, _i64p, _p, _i64, _i64, _i64, _i64,
                                           _i64, _p, _p, _p]),
    "cta_cuda_fma_gelu_deriv": (_int, [_p, _i64p, _p, _i64p, _p, _i64, _i64, _i64, _i64, _i64,
                                       _i64, _p, _p, _p, _p]),
    "cta_cuda_fma_gelu_tanh_deriv": (_int, [_p, _i64p, _p, _i64p, _p, _i64, _i64, _i64, _i64,
                                            _i64, _i64, _p, _p, _p, _p]),
    "cta_cuda_fma_mul": (_int, [_p, _i64p, _p, _i64p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p,
                                _p]),
    "cta_db_calculation_workspace": (_i64, [_i64, _i64, _i64]),
    "cta_db_calculation": (_int, [_p, _i64p, _i64, _i64, _i64, _p, _p, _p]),
    "cta_device_copy": (_int, [_p, _p, _i64, _p]),
    "cta_linear_weight_bias_grad_workspace": (_i64, [_i64, _i64, _i64]),
    "cta_linear_weight_bias_grad": (_int, [_p, _i64p, _p, _i64p, _i64, _i64, _i64, _p, _p, _p, _p]),
    "cta_gelu_fwd": (_int, [_p, _p, _i64, _p]),
    "cta_gelu_bwd": (_int, [_p, _p, _p, _i64, _p]),
    "cta_gelu_tanh_fwd": (_int, [_p, _p, _i64, _p]),
    "cta_gelu_tanh_bwd": (_int, [_p, _p, _p, _i64, _p]),
    "cta_softmax_fwd": (_int, [_p, _p, _i64, _i64, _p]),
    "cta_softmax_bwd": (_int, [_p, _p, _p, _i64, _i64, _p]),
    "cta_layernorm_fwd": (_int, [_p, _p, _p, _i64, _i64, _f32, _p, _p, _p, _p]),
    "cta_layernorm_bwd_workspace": (_i64, [_i64, _i64]),
    "cta_layernorm_bwd": (_int, [_p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p]),
    "cta_add_layernorm_fwd": (_int, [_p, _p, _p, _p, _i64, _i64, _f32, _p, _p, _p, _p, _p]),
    "cta_add_layernorm_bwd": (_int, [_p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p]),
    "cta_causal_self_attention_fwd": (_int, [_p, _i64, _i64, _i64, _i64, _int, _p, _p, _p]),
    "cta_causal_self_attention_bwd_workspace": (_i64, [_i64, _i64]),
    "cta_causal_self_attention_bwd": (_int, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _p, _i64p,
                                             _i64, _i64, _i64, _p, _p, _p, _p, _p]),
}


def declared_symbols(header: Path = HEADER) -> list[str]:
    """Function names declared in the public header."""
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(cta_[a-z0-9_]+)\s*\(", text)))


class CtaError(RuntimeError):
    pass


_lib = None


def lib() -> ctypes.CDLL:
    """Load the kernel library once and attach the prototypes."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH.name} is not built; run `python cuda_transformer_amd/build.py`")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def strides(values) -> ctypes.Array:
    arr = (ctypes.c_int64 * len(values))(*values)
    return arr


def call(name: str, *args) -> int:
    """Call an entry point; raise CtaError with the library's message on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    if isinstance(rc, int) and not name.endswith("_workspace") and rc != 0:
        raise CtaError(f"{name} failed ({rc}): {lib().cta_last_error().decode()}")
    return rc
