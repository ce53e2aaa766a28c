"""Linear-layer oracle.  TEST INFRASTRUCTURE ONLY (see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np


def fma_forward(x, weights, bias):
    """out[b] = x[b] @ W[b or 0] + bias (fused_multiply_add, Transformer_kernels/
    fused_multiply_add.cuh:10-92).  2-D weights are unsqueezed and a batch of 1 broadcasts
    (Transformer_launchers/linear_layer.cu:30-34)."""
    x = np.asarray(x)
    w = np.asarray(weights)
    if w.ndim == 2:
        w = w[None]
    return x @ w + np.asarray(bias)


def db_calculation(dy):
    """db[n] = sum over (batch, m) of dy (warp_sum_kernel, Transformer_kernels/
    warp_sum_kernel.cuh:13-51)."""
    return np.asarray(dy).sum(axis=(0, 1))


def linear_backward(x, weights, dy):
    """(dx, dW, db) as composed by CudaLinearLayer.backward (cuda_autograd_fns/
    cuda_linear_layer.py:14-29): dx = dy W^T, dW = sum_b x[b]^T dy[b], db = column sums."""
    x = np.asarray(x)
    dy = np.asarray(dy)
    w = np.asarray(weights)
    w3 = w[None] if w.ndim == 2 else w
    dx = dy @ np.swapaxes(w3, -1, -2)
    dw = (np.swapaxes(x, -1, -2) @ dy)
    if w.ndim == 2:
        dw = dw.sum(axis=0)
    return dx, dw, db_calculation(dy)


def mlp_forward(x, w1, b1, w2, b2):
    """The GPT MLP, fc1 -> exact GELU -> fc2 (gpt/gpt.py:133-136).  Returns (pre, h, out):
    fc1's pre-activation, its GELU and the fc2 output."""
    from .elementwise import gelu_forward

    pre = fma_forward(x, w1, b1)
    h = gelu_forward(pre)
    return pre, h, fma_forward(h, w2, b2)


def mlp_backward(x, w1, w2, pre, h, dz):
    """(dx, dW1, db1, dW2, db2): CudaLinearLayer.backward of fc2, CudaGeluLayer.backward and
    CudaLinearLayer.backward of fc1 in turn (cuda_linear_layer.py:14-29,
    cuda_gelu_layer.py:12-15)."""
    from .elementwise import gelu_backward

    dh, dw2, db2 = linear_backward(h, w2, dz)
    dpre = gelu_backward(pre, dh)
    dx, dw1, db1 = linear_backward(x, w1, dpre)
    return dx, dw1, db1, dw2, db2
