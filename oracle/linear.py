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
