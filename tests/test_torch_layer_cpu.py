"""The torch operator layer on the CPU: schemas, fake (meta) kernels, the reference's
Python API surface, and the absence of any CPU fallback."""
import pytest
import torch

import cuda_transformer
import cuda_transformer_amd
from cuda_transformer import ops

REFERENCE_ALL = [  # cuda_transformer/ops.py:4-10 of the reference
    "cuda_fma", "db_calculation", "cuda_softmax", "cuda_softmax_bwd", "gelu_activation",
    "gelu_activation_bwd", "causal_self_attention_fwd", "causal_self_attention_bwd",
    "flash_attention_fwd", "flash_attention_bwd",
]


def test_reference_api_surface():
    assert set(REFERENCE_ALL) <= set(ops.__all__)
    for name in REFERENCE_ALL + ["layernorm_fwd", "layernorm_bwd"]:
        assert callable(getattr(ops, name))
        assert hasattr(torch.ops.cuda_transformer, name)
    from cuda_autograd_fns import (CudaCausalSelfAttention, CudaFlashAttention,  # noqa: F401
                                   CudaGeluLayer, CudaLinearLayer, CudaSoftmaxLayer,
                                   cuda_flash_attention)
    assert cuda_flash_attention.CudaFlashAttention is CudaFlashAttention
    assert cuda_transformer._C is cuda_transformer_amd._C


def test_schemas_match_reference():
    schema = {name: str(getattr(torch.ops.cuda_transformer, name).default._schema)
              for name in REFERENCE_ALL}
    assert schema["flash_attention_fwd"] == (
        "cuda_transformer::flash_attention_fwd(Tensor Q, Tensor K, Tensor V, bool causal) "
        "-> (Tensor, Tensor)")
    assert schema["flash_attention_bwd"] == (
        "cuda_transformer::flash_attention_bwd(Tensor Q, Tensor K, Tensor V, Tensor O, "
        "Tensor dO, Tensor L, bool causal) -> (Tensor, Tensor, Tensor)")
    assert schema["cuda_fma"] == (
        "cuda_transformer::cuda_fma(Tensor x, Tensor weights, Tensor bias) -> Tensor")
    assert schema["causal_self_attention_fwd"] == (
        "cuda_transformer::causal_self_attention_fwd(Tensor qkv, int nh, bool causal) "
        "-> (Tensor, Tensor)")


def test_meta_shapes():
    m = dict(device="meta", dtype=torch.float32)
    q = torch.empty(2, 4, 100, 64, **m)
    O, L = ops.flash_attention_fwd(q, q, q, True)
    assert O.shape == q.shape and L.shape == (2, 4, 100)
    dq, dk, dv = ops.flash_attention_bwd(q, q, q, O, O, L, True)
    assert dq.shape == dk.shape == dv.shape == q.shape
    x = torch.empty(3, 10, 16, **m)
    assert ops.cuda_fma(x, torch.empty(16, 8, **m), torch.empty(8, **m)).shape == (3, 10, 8)
    assert ops.db_calculation(torch.empty(3, 10, 8, **m)).shape == (8,)
    from cuda_transformer_amd.ops import linear_weight_bias_grad
    dw, db = linear_weight_bias_grad(x, torch.empty(3, 10, 8, **m))
    assert dw.shape == (16, 8) and db.shape == (8,)
    assert ops.gelu_activation(x).shape == x.shape
    assert ops.gelu_activation_bwd(x, x).shape == x.shape
    assert ops.gelu_tanh_activation(x).shape == x.shape
    assert ops.gelu_tanh_activation_bwd(x, x).shape == x.shape
    pre, h = ops.cuda_fma_gelu_tanh(x, torch.empty(16, 8, **m), torch.empty(8, **m))
    assert pre.shape == h.shape == (3, 10, 8)
    assert ops.cuda_fma_gelu_tanh_grad(x, torch.empty(16, 8, **m), pre).shape == pre.shape
    for deriv_op in (ops.cuda_fma_gelu_deriv, ops.cuda_fma_gelu_tanh_deriv):
        d, h = deriv_op(x, torch.empty(16, 8, **m), torch.empty(8, **m))
        assert d.shape == h.shape == (3, 10, 8)
    assert ops.cuda_fma_mul(x, torch.empty(16, 8, **m), d).shape == d.shape
    assert ops.cuda_softmax(x).shape == x.shape
    out, probs = ops.causal_self_attention_fwd(torch.empty(2, 7, 96, **m), 4, True)
    assert out.shape == (2, 7, 32) and probs.shape == (2, 4, 7, 7)
    y, mean, rstd = ops.layernorm_fwd(x, torch.empty(16, **m), torch.empty(16, **m), 1e-5)
    assert y.shape == x.shape and mean.shape == rstd.shape == (3, 10)
    dx, dg, db = ops.layernorm_bwd(x, torch.empty(16, **m), mean, rstd, x)
    assert dx.shape == x.shape and dg.shape == db.shape == (16,)
    from cuda_transformer_amd.ops import add_layernorm_bwd, add_layernorm_fwd
    xs, y, mean, rstd = add_layernorm_fwd(x, x, torch.empty(16, **m), torch.empty(16, **m), 1e-5)
    assert xs.shape == y.shape == x.shape and mean.shape == rstd.shape == (3, 10)
    dx, dg, db = add_layernorm_bwd(xs, torch.empty(16, **m), mean, rstd, x, x)
    assert dx.shape == x.shape and dg.shape == db.shape == (16,)


def test_fake_rejects_wrong_dtype():
    q = torch.empty(1, 1, 8, 64, device="meta", dtype=torch.float64)
    with pytest.raises(Exception):
        ops.flash_attention_fwd(q, q, q, False)


def test_no_cpu_fallback():
    q = torch.randn(1, 1, 8, 64)
    with pytest.raises(NotImplementedError):
        ops.flash_attention_fwd(q, q, q, True)
    with pytest.raises(NotImplementedError):
        ops.cuda_fma(torch.randn(1, 2, 3), torch.randn(3, 4), torch.randn(4))
    with pytest.raises(NotImplementedError):
        ops.gelu_tanh_activation(torch.randn(2, 3, 4))


def test_bwd_workspace_cap_setting():
    """The dS workspace cap of flash_attention_bwd: 8 GiB by default, settable (returns the
    previous value), byte counts only."""
    _C = cuda_transformer_amd._C
    assert _C.bwd_workspace_cap() == 8 << 30
    assert _C.set_bwd_workspace_cap(0) == 8 << 30
    try:
        assert _C.bwd_workspace_cap() == 0
        with pytest.raises(ValueError):
            _C.set_bwd_workspace_cap(-5)
        with pytest.raises(TypeError):
            _C.set_bwd_workspace_cap("1 GiB")
        assert _C.bwd_workspace_cap() == 0
    finally:
        assert _C.set_bwd_workspace_cap(8 << 30) == 0
