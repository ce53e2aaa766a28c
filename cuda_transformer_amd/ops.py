"""Python wrappers of the ``cuda_transformer`` operators, with fake (meta) kernels.

Mirrors the reference's cuda_transformer/ops.py:1-138: the same ten functions, calling
``torch.ops.cuda_transformer.<op>.default`` and registering ``torch.library.register_fake``
shape functions for FakeTensor / ``torch.compile`` tracing.  Two deviations, both fixes:

* the fake of ``gelu_activation_bwd`` checks ``dy.dtype`` (ops.py:73 reads ``dy.type``, which
  is a method and never equals ``torch.float32``);
* the fake of ``causal_self_attention_fwd`` returns probs of shape (B, nh, T, T) — the real
  operator's shape (causal_self_attn_layer.cu:36) — where ops.py:81-89 says (B, T, T).

Added: ``layernorm_fwd`` / ``layernorm_bwd`` (the reference's LayerNorm is plain torch,
gpt/gpt.py:47-59), and ``cuda_fma_gelu`` / ``cuda_fma_gelu_grad``, the GPT MLP's linear+GELU
pairs (gpt/gpt.py:134-135 and their backward) fused into one GEMM each, and
``gelu_tanh_activation`` / ``gelu_tanh_activation_bwd``, the tanh-approximated GELU (with its
fused linear pair ``cuda_fma_gelu_tanh`` / ``cuda_fma_gelu_tanh_grad``).
"""
import torch
from torch import Tensor

__all__ = [
    "cuda_fma", "db_calculation", "linear_weight_bias_grad", "cuda_fma_gelu", "cuda_fma_gelu_grad", "cuda_fma_gelu_tanh",
    "cuda_fma_gelu_tanh_grad", "cuda_fma_gelu_deriv", "cuda_fma_gelu_tanh_deriv", "cuda_fma_mul",
    "cuda_softmax", "cuda_softmax_bwd",
    "gelu_activation", "gelu_activation_bwd", "gelu_tanh_activation", "gelu_tanh_activation_bwd",
    "causal_self_attention_fwd", "causal_self_attention_bwd",
    "flash_attention_fwd", "flash_attention_bwd",
    "flash_attention_qkv_fwd", "flash_attention_qkv_bwd",
    "layernorm_fwd", "layernorm_bwd", "add_layernorm_fwd", "add_layernorm_bwd",
]

_ops = torch.ops.cuda_transformer


def _f32(*ts):
    for t in ts:
        torch._check(t.dtype == torch.float32)


def _same_device(*ts):
    torch._check(all(t.device == ts[0].device for t in ts))


# ----------------------------------------------------------------- linear layer
def cuda_fma(x: Tensor, weights: Tensor, bias: Tensor) -> Tensor:
    """out[b] = x[b] @ weights[b or 0] + bias  (reference ops.py:13-15)."""
    return _ops.cuda_fma.default(x, weights, bias)


@torch.library.register_fake("cuda_transformer::cuda_fma")
def _(x, weights, bias):
    _f32(x, weights, bias)
    _same_device(x, weights, bias)
    w = weights if weights.dim() == 3 else weights.unsqueeze(0)
    return torch.empty(x.size(0), x.size(1), w.size(2), dtype=x.dtype, device=x.device)


def cuda_fma_gelu(x: Tensor, weights: Tensor, bias: Tensor) -> tuple[Tensor, Tensor]:
    """(pre, out) with pre = x @ weights + bias and out = gelu(pre), from one GEMM.

    Bitwise equal to ``cuda_fma`` followed by ``gelu_activation``."""
    return _ops.cuda_fma_gelu.default(x, weights, bias)


@torch.library.register_fake("cuda_transformer::cuda_fma_gelu")
def _(x, weights, bias):
    _f32(x, weights, bias)
    _same_device(x, weights, bias)
    w = weights if weights.dim() == 3 else weights.unsqueeze(0)
    shape = (x.size(0), x.size(1), w.size(2))
    return (torch.empty(shape, dtype=x.dtype, device=x.device),
            torch.empty(shape, dtype=x.dtype, device=x.device))


def cuda_fma_gelu_grad(dy: Tensor, weights: Tensor, pre: Tensor) -> Tensor:
    """(dy @ weights) * gelu'(pre), from one GEMM.

    Bitwise equal to ``cuda_fma`` with a zero bias followed by ``gelu_activation_bwd(pre, .)``."""
    return _ops.cuda_fma_gelu_grad.default(dy, weights, pre)


@torch.library.register_fake("cuda_transformer::cuda_fma_gelu_grad")
def _(dy, weights, pre):
    _f32(dy, weights, pre)
    _same_device(dy, weights, pre)
    return torch.empty(pre.shape, dtype=dy.dtype, device=dy.device)


def cuda_fma_gelu_tanh(x: Tensor, weights: Tensor, bias: Tensor) -> tuple[Tensor, Tensor]:
    """As ``cuda_fma_gelu`` with the tanh-approximated GELU: bitwise equal to ``cuda_fma``
    followed by ``gelu_tanh_activation``."""
    return _ops.cuda_fma_gelu_tanh.default(x, weights, bias)


@torch.library.register_fake("cuda_transformer::cuda_fma_gelu_tanh")
def _(x, weights, bias):
    _f32(x, weights, bias)
    _same_device(x, weights, bias)
    w = weights if weights.dim() == 3 else weights.unsqueeze(0)
    shape = (x.size(0), x.size(1), w.size(2))
    return (torch.empty(shape, dtype=x.dtype, device=x.device),
            torch.empty(shape, dtype=x.dtype, device=x.device))


def cuda_fma_gelu_tanh_grad(dy: Tensor, weights: Tensor, pre: Tensor) -> Tensor:
    """As ``cuda_fma_gelu_grad`` with the tanh-approximated GELU: bitwise equal to ``cuda_fma``
    with a zero bias followed by ``gelu_tanh_activation_bwd(pre, .)``."""
    return _ops.cuda_fma_gelu_tanh_grad.default(dy, weights, pre)


@torch.library.register_fake("cuda_transformer::cuda_fma_gelu_tanh_grad")
def _(dy, weights, pre):
    _f32(dy, weights, pre)
    _same_device(dy, weights, pre)
    return torch.empty(pre.shape, dtype=dy.dtype, device=dy.device)


def cuda_fma_gelu_deriv(x: Tensor, weights: Tensor, bias: Tensor) -> tuple[Tensor, Tensor]:
    """(deriv, out) with deriv = gelu'(x @ weights + bias) and out = gelu(x @ weights + bias),
    from one GEMM; ``cuda_fma_mul(dy, w, deriv)`` is then bitwise equal to
    ``cuda_fma_gelu_grad(dy, w, pre)``."""
    return _ops.cuda_fma_gelu_deriv.default(x, weights, bias)


def cuda_fma_gelu_tanh_deriv(x: Tensor, weights: Tensor, bias: Tensor) -> tuple[Tensor, Tensor]:
    """As ``cuda_fma_gelu_deriv`` with the tanh-approximated GELU (pairs with
    ``cuda_fma_gelu_tanh_grad``)."""
    return _ops.cuda_fma_gelu_tanh_deriv.default(x, weights, bias)


def cuda_fma_mul(dy: Tensor, weights: Tensor, d: Tensor) -> Tensor:
    """(dy @ weights) * d, from one GEMM (d of the output's shape)."""
    return _ops.cuda_fma_mul.default(dy, weights, d)


for _name in ("cuda_fma_gelu_deriv", "cuda_fma_gelu_tanh_deriv"):
    @torch.library.register_fake(f"cuda_transformer::{_name}")
    def _(x, weights, bias):
        _f32(x, weights, bias)
        _same_device(x, weights, bias)
        w = weights if weights.dim() == 3 else weights.unsqueeze(0)
        shape = (x.size(0), x.size(1), w.size(2))
        return (torch.empty(shape, dtype=x.dtype, device=x.device),
                torch.empty(shape, dtype=x.dtype, device=x.device))


@torch.library.register_fake("cuda_transformer::cuda_fma_mul")
def _(dy, weights, d):
    _f32(dy, weights, d)
    _same_device(dy, weights, d)
    return torch.empty(d.shape, dtype=dy.dtype, device=dy.device)


def db_calculation(dy: Tensor) -> Tensor:
    """Bias gradient: sum of dy over (batch, rows)  (reference ops.py:26-28)."""
    return _ops.db_calculation.default(dy)


@torch.library.register_fake("cuda_transformer::db_calculation")
def _(dy):
    _f32(dy)
    return torch.empty(dy.size(-1), dtype=dy.dtype, device=dy.device)


def linear_weight_bias_grad(x: Tensor, dy: Tensor):
    """(dW, db) = (x^T dy, column sums of dy) over every row of x (..., k) and dy (..., n):
    ``cuda_fma`` on the x^T view (zero bias) and ``db_calculation`` in one GEMM whose dy slices
    also feed the column sums.  dW is bitwise equal to the ``cuda_fma`` route; db matches
    ``db_calculation`` up to summation order.  No reference op (the reference makes the two
    calls, cuda_linear_layer.py:21-27)."""
    return _ops.linear_weight_bias_grad.default(x, dy)


@torch.library.register_fake("cuda_transformer::linear_weight_bias_grad")
def _(x, dy):
    _f32(x, dy)
    _same_device(x, dy)
    torch._check(x.dim() == dy.dim() and x.shape[:-1] == dy.shape[:-1],
                 lambda: "x and dy must agree in every dim but the last")
    return (torch.empty(x.size(-1), dy.size(-1), dtype=dy.dtype, device=dy.device),
            torch.empty(dy.size(-1), dtype=dy.dtype, device=dy.device))


# ----------------------------------------------------------------- softmax
def cuda_softmax(x: Tensor) -> Tensor:
    """Row softmax over the last dim of a 3-D tensor  (reference ops.py:36-38)."""
    return _ops.cuda_softmax.default(x)


@torch.library.register_fake("cuda_transformer::cuda_softmax")
def _(x):
    _f32(x)
    return torch.empty_like(x)


def cuda_softmax_bwd(probs: Tensor, dp: Tensor) -> Tensor:
    """dx = probs * (dp - sum(probs * dp))  (reference ops.py:45-47)."""
    return _ops.cuda_softmax_bwd.default(probs, dp)


@torch.library.register_fake("cuda_transformer::cuda_softmax_bwd")
def _(probs, dp):
    _f32(probs, dp)
    _same_device(probs, dp)
    return torch.empty_like(probs)


# ----------------------------------------------------------------- GELU
def gelu_activation(x: Tensor) -> Tensor:
    """Exact (erf) GELU  (reference ops.py:56-58)."""
    return _ops.gelu_activation.default(x)


@torch.library.register_fake("cuda_transformer::gelu_activation")
def _(x):
    _f32(x)
    return torch.empty_like(x)


def gelu_activation_bwd(x: Tensor, dy: Tensor) -> Tensor:
    """GELU input gradient  (reference ops.py:66-68)."""
    return _ops.gelu_activation_bwd.default(x, dy)


@torch.library.register_fake("cuda_transformer::gelu_activation_bwd")
def _(x, dy):
    _f32(x, dy)
    _same_device(x, dy)
    return torch.empty_like(x)


# ----------------------------------------------------------------- tanh GELU
def gelu_tanh_activation(x: Tensor) -> Tensor:
    """tanh-approximated GELU, ``F.gelu(x, approximate="tanh")``.  New op: the reference's GELU
    is erf-exact (GeLU.cuh:7-16); this is the GPT-2 form, for models that use it."""
    return _ops.gelu_tanh_activation.default(x)


@torch.library.register_fake("cuda_transformer::gelu_tanh_activation")
def _(x):
    _f32(x)
    return torch.empty_like(x)


def gelu_tanh_activation_bwd(x: Tensor, dy: Tensor) -> Tensor:
    """Input gradient of ``gelu_tanh_activation`` (torch's tanh-GELU backward)."""
    return _ops.gelu_tanh_activation_bwd.default(x, dy)


@torch.library.register_fake("cuda_transformer::gelu_tanh_activation_bwd")
def _(x, dy):
    _f32(x, dy)
    _same_device(x, dy)
    return torch.empty_like(x)


# ----------------------------------------------------------------- naive attention
def causal_self_attention_fwd(qkv: Tensor, nh: int, causal: bool) -> tuple[Tensor, Tensor]:
    """Materialised attention over packed qkv (B, T, 3C) -> (out, probs)  (ops.py:78-80)."""
    return _ops.causal_self_attention_fwd.default(qkv, nh, causal)


@torch.library.register_fake("cuda_transformer::causal_self_attention_fwd")
def _(qkv, nh, causal):
    _f32(qkv)
    b, t, three_c = qkv.shape
    c = three_c // 3
    out = torch.empty((b, t, c), dtype=qkv.dtype, device=qkv.device)
    probs = torch.empty((b, nh, t, t), dtype=qkv.dtype, device=qkv.device)
    return out, probs


def causal_self_attention_bwd(Q: Tensor, K: Tensor, V: Tensor, probs: Tensor, dO: Tensor):
    """Naive attention backward on (B*nh, T, hs); dq, dk unscaled  (ops.py:91-93)."""
    return _ops.causal_self_attention_bwd.default(Q, K, V, probs, dO)


@torch.library.register_fake("cuda_transformer::causal_self_attention_bwd")
def _(Q, K, V, probs, dO):
    _f32(Q, K, V, probs, dO)
    _same_device(Q, K, V, probs, dO)
    return torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)


# ----------------------------------------------------------------- FlashAttention-2
def flash_attention_fwd(Q: Tensor, K: Tensor, V: Tensor, causal: bool) -> tuple[Tensor, Tensor]:
    """FA2 forward -> (O, L), L = rowmax + ln(rowsum)  (reference ops.py:109-111).

    Extension: bfloat16 or float16 Q, K, V (hs 32, 64 or 128) run the 16-bit kernel, which returns
    O in the input dtype and L in float32; the reference's kernels are float32 only."""
    return _ops.flash_attention_fwd.default(Q, K, V, causal)


@torch.library.register_fake("cuda_transformer::flash_attention_fwd")
def _(Q, K, V, causal):
    if Q.dtype in (torch.bfloat16, torch.float16):
        torch._check(K.dtype == Q.dtype and V.dtype == Q.dtype,
                     lambda: "Q, K and V must have the same dtype")
    else:
        _f32(Q, K, V)
    _same_device(Q, K, V)
    O = torch.empty((Q.size(0), Q.size(1), Q.size(2), Q.size(3)), dtype=Q.dtype, device=Q.device)
    L = torch.empty((Q.size(0), Q.size(1), Q.size(2)), dtype=torch.float32, device=Q.device)
    return O, L


def flash_attention_bwd(Q: Tensor, K: Tensor, V: Tensor, O: Tensor, dO: Tensor, L: Tensor,
                        causal: bool):
    """FA2 backward -> (dQ, dK, dV)  (reference ops.py:123-125).

    Extension: bfloat16 or float16 Q, K, V, O, dO with float32 L (hs 32, 64 or 128) run the 16-bit
    kernels and return gradients in the input dtype."""
    return _ops.flash_attention_bwd.default(Q, K, V, O, dO, L, causal)


@torch.library.register_fake("cuda_transformer::flash_attention_bwd")
def _(Q, K, V, O, dO, L, causal):
    if Q.dtype in (torch.bfloat16, torch.float16):
        torch._check(all(t.dtype == Q.dtype for t in (K, V, O, dO)),
                     lambda: "Q, K, V, O and dO must have the same dtype")
        _f32(L)
    else:
        _f32(Q, K, V, O, dO, L)
    _same_device(Q, K, V, O, dO, L)
    return torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)


# ----------------------------------------------------------------- packed-qkv FA2 (added)
def flash_attention_qkv_fwd(qkv: Tensor, nh: int, causal: bool) -> tuple[Tensor, Tensor]:
    """FA2 forward on a packed (B, T, 3C) projection -> (out (B, T, C), L (B, nh, T)).

    Q, K, V are qkv's three column blocks with head h in columns h*hs .. h*hs + hs - 1 (the
    slicing of gpt/gpt.py:104-107); out holds O in the same head-interleaved order.  The same
    kernel as flash_attention_fwd on the head views, read and written in place (no transposes)."""
    return _ops.flash_attention_qkv_fwd.default(qkv, nh, causal)


@torch.library.register_fake("cuda_transformer::flash_attention_qkv_fwd")
def _(qkv, nh, causal):
    _f32(qkv)
    torch._check(qkv.dim() == 3 and qkv.size(2) % (3 * nh) == 0,
                 lambda: "qkv.size(2) must be 3 * nh * hs")
    B, T, C = qkv.size(0), qkv.size(1), qkv.size(2) // 3
    out = torch.empty((B, T, C), dtype=qkv.dtype, device=qkv.device)
    L = torch.empty((B, nh, T), dtype=torch.float32, device=qkv.device)
    return out, L


def flash_attention_qkv_bwd(qkv: Tensor, out: Tensor, dout: Tensor, L: Tensor, nh: int,
                            causal: bool) -> Tensor:
    """FA2 backward of flash_attention_qkv_fwd -> d(qkv) (B, T, 3C), the gradients of the three
    column blocks written in place of one another's concatenation."""
    return _ops.flash_attention_qkv_bwd.default(qkv, out, dout, L, nh, causal)


@torch.library.register_fake("cuda_transformer::flash_attention_qkv_bwd")
def _(qkv, out, dout, L, nh, causal):
    _f32(qkv, out, dout, L)
    _same_device(qkv, out, dout, L)
    return torch.empty_like(qkv, memory_format=torch.contiguous_format)


# ----------------------------------------------------------------- LayerNorm (added)
def layernorm_fwd(x: Tensor, gamma: Tensor, beta: Tensor, eps: float = 1e-5):
    """LayerNorm over the last dim -> (y, mean, rstd); semantics of gpt/gpt.py:47-59."""
    return _ops.layernorm_fwd.default(x, gamma, beta, eps)


@torch.library.register_fake("cuda_transformer::layernorm_fwd")
def _(x, gamma, beta, eps):
    _f32(x, gamma, beta)
    _same_device(x, gamma, beta)
    stat = torch.empty(x.shape[:-1], dtype=x.dtype, device=x.device)
    return torch.empty_like(x), stat, torch.empty_like(stat)


def layernorm_bwd(x: Tensor, gamma: Tensor, mean: Tensor, rstd: Tensor, dy: Tensor):
    """LayerNorm backward -> (dx, dgamma, dbeta)."""
    return _ops.layernorm_bwd.default(x, gamma, mean, rstd, dy)


@torch.library.register_fake("cuda_transformer::layernorm_bwd")
def _(x, gamma, mean, rstd, dy):
    _f32(x, gamma, mean, rstd, dy)
    _same_device(x, gamma, mean, rstd, dy)
    n = x.size(-1)
    return (torch.empty_like(x), torch.empty(n, dtype=x.dtype, device=x.device),
            torch.empty(n, dtype=x.dtype, device=x.device))


def add_layernorm_fwd(x: Tensor, f: Tensor, gamma: Tensor, beta: Tensor, eps: float = 1e-5):
    """Residual add fused with the LayerNorm after it -> (xsum = x + f, LayerNorm(xsum), mean,
    rstd): the bits of ``x + f`` followed by ``layernorm_fwd``, in one pass.  No reference op
    (the pre-LN block's residual adds and LayerNorms, gpt/gpt.py:147-150)."""
    return _ops.add_layernorm_fwd.default(x, f, gamma, beta, eps)


@torch.library.register_fake("cuda_transformer::add_layernorm_fwd")
def _(x, f, gamma, beta, eps):
    _f32(x, f, gamma, beta)
    _same_device(x, f, gamma, beta)
    stat = torch.empty(x.shape[:-1], dtype=x.dtype, device=x.device)
    return torch.empty_like(x), torch.empty_like(x), stat, torch.empty_like(stat)


def add_layernorm_bwd(xsum: Tensor, gamma: Tensor, mean: Tensor, rstd: Tensor, dy: Tensor,
                      dres: Tensor):
    """Backward of ``add_layernorm_fwd`` -> (dx, dgamma, dbeta) with dx = LayerNorm backward of
    dy at xsum plus dres, the gradient reaching xsum by the residual path (the gradient of both
    x and f): the bits of ``layernorm_bwd`` followed by ``+ dres``."""
    return _ops.add_layernorm_bwd.default(xsum, gamma, mean, rstd, dy, dres)


@torch.library.register_fake("cuda_transformer::add_layernorm_bwd")
def _(xsum, gamma, mean, rstd, dy, dres):
    _f32(xsum, gamma, mean, rstd, dy, dres)
    _same_device(xsum, gamma, mean, rstd, dy, dres)
    n = xsum.size(-1)
    return (torch.empty_like(xsum), torch.empty(n, dtype=xsum.dtype, device=xsum.device),
            torch.empty(n, dtype=xsum.dtype, device=xsum.device))
