"""GELU, softmax and LayerNorm oracles.  TEST INFRASTRUCTURE ONLY (see oracle/__init__.py)."""
from __future__ import annotations

import math

import numpy as np

try:  # scipy's erf is a vectorised library routine; math.erf is the scalar fallback
    from scipy.special import erf as _erf
except Exception:  # pragma: no cover
    _erf = np.vectorize(math.erf, otypes=[np.float64])

INV_SQRT2 = 1.0 / math.sqrt(2.0)
INV_SQRT_2PI = 1.0 / math.sqrt(2.0 * math.pi)


def normal_cdf(x):
    """Phi(x) = (1 + erf(x / sqrt 2)) / 2 (the normcdff of GeLU.cuh:14,28)."""
    return 0.5 * (1.0 + _erf(np.asarray(x, dtype=np.float64) * INV_SQRT2))


def gelu_forward(x):
    """y = x Phi(x) — exact GELU (Transformer_kernels/GeLU.cuh:7-16)."""
    x = np.asarray(x, dtype=np.float64)
    return x * normal_cdf(x)


def gelu_backward(x, dy):
    """dx = dy (Phi(x) + x phi(x)), phi(x) = e^{-x^2/2} / sqrt(2 pi) (GeLU.cuh:19-29)."""
    x = np.asarray(x, dtype=np.float64)
    pdf = INV_SQRT_2PI * np.exp(-0.5 * x * x)
    return np.asarray(dy, dtype=np.float64) * (normal_cdf(x) + x * pdf)


SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)
GELU_CUBIC = 0.044715


def gelu_tanh_forward(x):
    """y = x (1 + tanh u) / 2, u = sqrt(2/pi) (x + 0.044715 x^3): the tanh-approximated GELU of
    the non-attention benchmark workload (torch's F.gelu(x, approximate="tanh")).  The reference
    has no kernel for it; its GELU is erf-exact (GeLU.cuh:7-16)."""
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + np.tanh(SQRT_2_OVER_PI * (x + GELU_CUBIC * x**3)))


def gelu_tanh_backward(x, dy):
    """dx = dy ((1 + tanh u) / 2 + x (1 - tanh^2 u) u' / 2), u' = sqrt(2/pi)(1 + 3 0.044715 x^2)."""
    x = np.asarray(x, dtype=np.float64)
    t = np.tanh(SQRT_2_OVER_PI * (x + GELU_CUBIC * x**3))
    du = SQRT_2_OVER_PI * (1.0 + 3.0 * GELU_CUBIC * x * x)
    return np.asarray(dy, dtype=np.float64) * (0.5 * (1.0 + t) + 0.5 * x * (1.0 - t * t) * du)


def softmax_forward(x):
    """Row softmax over the last axis: max pass, sum of e^{x - max}, then e^{x - max} * (1/sum)
    (naive_softmax, Transformer_kernels/softmax.cuh:25-106)."""
    x = np.asarray(x)
    with np.errstate(invalid="ignore"):
        m = x.max(axis=-1, keepdims=True)
        e = np.exp(x - m)
        return e * (1.0 / e.sum(axis=-1, keepdims=True))


def softmax_backward(p, dp):
    """dx = p (dp - sum(p dp)) per row (naive_softmax_bwd, softmax.cuh:108-159)."""
    p = np.asarray(p)
    dp = np.asarray(dp)
    return p * (dp - (p * dp).sum(axis=-1, keepdims=True))


def layernorm_forward(x, gamma, beta, eps: float = 1e-5):
    """y = (x - mean) / sqrt(var + eps) * gamma + beta, biased variance over the last axis
    (LayerNorm.forward, gpt/gpt.py:54-59).  Returns (y, mean, rstd)."""
    x = np.asarray(x)
    mean = x.mean(axis=-1)
    var = ((x - mean[..., None]) ** 2).mean(axis=-1)
    rstd = 1.0 / np.sqrt(var + eps)
    y = (x - mean[..., None]) * rstd[..., None] * gamma + beta
    return y, mean, rstd


def layernorm_backward(x, gamma, mean, rstd, dy):
    """Gradient of layernorm_forward (the reference differentiates gpt.py:54-59 with torch
    autograd): xh = (x - mean) rstd, g = dy gamma,
    dx = rstd (g - mean(g) - xh mean(g xh)), dgamma = sum dy xh, dbeta = sum dy."""
    x = np.asarray(x)
    dy = np.asarray(dy)
    xh = (x - mean[..., None]) * rstd[..., None]
    g = dy * gamma
    dx = rstd[..., None] * (g - g.mean(axis=-1, keepdims=True)
                            - xh * (g * xh).mean(axis=-1, keepdims=True))
    red = tuple(range(x.ndim - 1))
    return dx, (dy * xh).sum(axis=red), dy.sum(axis=red)
