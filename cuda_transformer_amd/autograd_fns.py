"""``torch.autograd.Function`` wrappers over the ``cuda_transformer`` operators.

Same classes, ``apply`` signatures and saved tensors as the reference's cuda_autograd_fns/
(cuda_flash_attention.py:4-17, cuda_linear_layer.py:4-28, cuda_gelu_layer.py:4-14,
cuda_softmax_layer.py:4-15, cuda_causal_self_attention.py:4-35), plus ``CudaLayerNorm``,
``CudaMLP`` (the GPT MLP with its GELU folded into the GEMM epilogues), ``CudaGeluTanhLayer``
(the tanh-approximated GELU), ``CudaFlashAttentionQKV`` (attention on a packed qkv projection,
no head transposes), ``CudaAddLayerNorm`` (a residual add fused with the next LayerNorm) and
``CudaEmbedding`` (token + position embedding whose backward never waits on the host).

Deviations, each a fix:

* ``CudaCausalSelfAttention.backward`` scales dq and dk by 1/sqrt(hs).  The reference scales
  dk and dv (cuda_causal_self_attention.py:34), which gives wrong dq and dv; its own test
  scales dq and dk (test/test_causal_self_attn.py:67).
* ``CudaLinearLayer.backward`` allocates its zero bias on dy's device instead of the
  hard-coded 'cuda' device, and computes dW as one GEMM over the flattened (batch*m) axis
  instead of a per-batch GEMM followed by ``torch.sum(dim=0)`` (same sum, fewer bytes).  With
  2-D weights that GEMM also produces db (``linear_weight_bias_grad``): dy is read once.
  Its zero bias is one cached read-only tensor per (length, dtype, device) rather than a new
  ``torch.zeros`` (a fill launch) on every backward.
"""
import torch
import torch.nn.functional as F

from .ops import (
    causal_self_attention_bwd, causal_self_attention_fwd, cuda_fma, cuda_fma_gelu_deriv,
    cuda_fma_gelu_tanh_deriv, cuda_fma_mul, cuda_softmax, cuda_softmax_bwd, db_calculation, flash_attention_bwd, flash_attention_fwd, flash_attention_qkv_bwd, flash_attention_qkv_fwd, gelu_activation,
    gelu_activation_bwd, gelu_tanh_activation, gelu_tanh_activation_bwd, layernorm_bwd, layernorm_fwd,
    linear_weight_bias_grad, add_layernorm_bwd, add_layernorm_fwd,
)

__all__ = [
    "CudaCausalSelfAttention", "CudaFlashAttention", "CudaGeluLayer", "CudaLinearLayer",
    "CudaSoftmaxLayer", "CudaLayerNorm", "CudaMLP", "CudaGeluTanhLayer", "CudaFlashAttentionQKV",
    "CudaAddLayerNorm", "CudaEmbedding",
]


_ZEROS = {}


def _zeros(n, like):
    """A length-n zero vector on like's device and dtype, allocated once and never written:
    the zero bias of the backward GEMMs.  Under stream capture a first use allocates a plain
    zeros tensor instead: memory from the graph's private pool must not outlive the graph."""
    key = (n, like.dtype, like.device)
    z = _ZEROS.get(key)
    if z is None:
        z = torch.zeros(n, dtype=like.dtype, device=like.device)
        if not (like.is_cuda and torch.cuda.is_current_stream_capturing()):
            _ZEROS[key] = z
    return z


class CudaFlashAttention(torch.autograd.Function):
    """(q, k, v, causal) -> (o, l); backward ignores grad_l (cuda_flash_attention.py:4-17)."""

    @staticmethod
    def forward(ctx, q, k, v, causal):
        o, l = flash_attention_fwd(q, k, v, causal)
        ctx.save_for_backward(q, k, v, o, l)
        ctx.causal = causal
        return o, l

    @staticmethod
    def backward(ctx, grad_output, grad_l=None):
        q, k, v, o, l = ctx.saved_tensors
        dq, dk, dv = flash_attention_bwd(q, k, v, o, grad_output, l, ctx.causal)
        return dq, dk, dv, None


class CudaFlashAttentionQKV(torch.autograd.Function):
    """(qkv (B, T, 3C), nh, causal) -> attention output (B, T, C), heads interleaved as in qkv:
    the reference GPT's qkv.split -> head views -> flash attention -> transpose back
    (gpt/gpt.py:104-109), with the kernels reading and writing the packed layouts in place."""

    @staticmethod
    def forward(ctx, qkv, nh, causal):
        out, l = flash_attention_qkv_fwd(qkv, nh, causal)
        ctx.save_for_backward(qkv, out, l)
        ctx.nh, ctx.causal = nh, causal
        return out

    @staticmethod
    def backward(ctx, grad_output):
        qkv, out, l = ctx.saved_tensors
        return flash_attention_qkv_bwd(qkv, out, grad_output, l, ctx.nh, ctx.causal), None, None


class CudaLinearLayer(torch.autograd.Function):
    """(x, weights (k, n) or (b, k, n), bias (n)) -> x @ W + b (cuda_linear_layer.py:4-28)."""

    @staticmethod
    def forward(ctx, x, weights, bias):
        out = cuda_fma(x, weights, bias)
        ctx.save_for_backward(x, weights, bias, out)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        x, weights, _, _ = ctx.saved_tensors
        dy = grad_output
        w = weights.unsqueeze(0) if weights.dim() == 2 else weights
        dx = cuda_fma(dy, w.transpose(1, 2), _zeros(x.shape[-1], dy))
        dw, db = _weight_and_bias_grads(x, weights, dy)
        return dx, dw, db


def _weight_and_bias_grads(x, weights, dy):
    """dW = sum_b x[b]^T dy[b] and db = sum of dy over (batch, rows) (cuda_linear_layer.py:21-27)."""
    if weights.dim() == 2:
        # sum_b x[b]^T dy[b] == (x as (b*m, k))^T (dy as (b*m, n)): one GEMM, K = b*m, which
        # also sums dy's columns for db as it streams them
        return linear_weight_bias_grad(x, dy)
    dw = cuda_fma(x.transpose(1, 2), dy, _zeros(dy.shape[-1], dy))
    return dw, db_calculation(dy)


class CudaGeluLayer(torch.autograd.Function):
    """Exact GELU (cuda_gelu_layer.py:4-14)."""

    @staticmethod
    def forward(ctx, x):
        out = gelu_activation(x)
        ctx.save_for_backward(x)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        (x,) = ctx.saved_tensors
        return gelu_activation_bwd(x, grad_output.contiguous())


class CudaGeluTanhLayer(torch.autograd.Function):
    """tanh-approximated GELU, ``F.gelu(x, approximate="tanh")``; same saved tensor and
    backward shape as ``CudaGeluLayer``.  No reference class (its GELU is erf-exact)."""

    @staticmethod
    def forward(ctx, x):
        out = gelu_tanh_activation(x)
        ctx.save_for_backward(x)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        (x,) = ctx.saved_tensors
        return gelu_tanh_activation_bwd(x, grad_output.contiguous())


class CudaMLP(torch.autograd.Function):
    """(x, w1, b1, w2, b2) -> gelu(x @ w1 + b1) @ w2 + b2, the GPT MLP (gpt/gpt.py:133-136).

    Same values, bit for bit, as CudaLinearLayer, CudaGeluLayer and CudaLinearLayer applied in
    turn (2-D weights), in fewer passes over the (batch, m, 4 d_model) hidden tensor: the
    forward's fc1 GEMM writes GELU(pre) and GELU'(pre) together (``cuda_fma_gelu_deriv``:
    its epilogue already holds the normal CDF that both need), and the backward's fc2 dx GEMM
    multiplies its product by the saved derivative before the store (``cuda_fma_mul``), so
    neither GELU pass re-reads the hidden tensor and the backward product carries no GELU
    arithmetic.  The saved derivative takes the place of the pre-activation (same memory).

    An optional sixth argument ``tanh=True`` selects the tanh-approximated GELU (the GPT-2
    form; ``CudaGeluTanhLayer`` in the composition above).
    """

    @staticmethod
    def forward(ctx, x, w1, b1, w2, b2, tanh=False):
        torch._check(w1.dim() == 2 and w2.dim() == 2, lambda: "CudaMLP takes 2-D weights")
        deriv, h = (cuda_fma_gelu_tanh_deriv if tanh else cuda_fma_gelu_deriv)(x, w1, b1)
        out = cuda_fma(h, w2, b2)
        ctx.save_for_backward(x, w1, w2, deriv, h)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        x, w1, w2, deriv, h = ctx.saved_tensors
        dz = grad_output
        dw2, db2 = _weight_and_bias_grads(h, w2, dz)
        dpre = cuda_fma_mul(dz, w2.unsqueeze(0).transpose(1, 2), deriv)
        dw1, db1 = _weight_and_bias_grads(x, w1, dpre)
        dx = cuda_fma(dpre, w1.unsqueeze(0).transpose(1, 2), _zeros(x.shape[-1], dz))
        return dx, dw1, db1, dw2, db2, None


class CudaSoftmaxLayer(torch.autograd.Function):
    """Row softmax over the last dim of a 3-D tensor (cuda_softmax_layer.py:4-15)."""

    @staticmethod
    def forward(ctx, x):
        out = cuda_softmax(x)
        ctx.save_for_backward(out)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        (out,) = ctx.saved_tensors
        return cuda_softmax_bwd(out, grad_output.contiguous())


class CudaCausalSelfAttention(torch.autograd.Function):
    """Materialised attention over packed qkv (cuda_causal_self_attention.py:4-35)."""

    @staticmethod
    def forward(ctx, qkv, nh, causal):
        out, probs = causal_self_attention_fwd(qkv, nh, causal)
        ctx.save_for_backward(qkv, probs)
        ctx.nh = nh
        return out

    @staticmethod
    def backward(ctx, grad_output):
        qkv, probs = ctx.saved_tensors
        nh = ctx.nh
        q, k, v = qkv.chunk(3, dim=-1)
        B, T, C = q.shape
        hs = C // nh

        def heads(t):
            return t.reshape(B, T, nh, hs).transpose(1, 2).reshape(B * nh, T, hs)

        def unheads(t):
            return t.reshape(B, nh, T, hs).transpose(1, 2).reshape(B, T, C)

        dq, dk, dv = causal_self_attention_bwd(
            heads(q), heads(k), heads(v), probs.reshape(B * nh, T, T),
            heads(grad_output.contiguous()))
        sm_scale = hs ** 0.5
        grads = torch.cat([unheads(dq) / sm_scale, unheads(dk) / sm_scale, unheads(dv)], dim=-1)
        return grads, None, None


class CudaAddLayerNorm(torch.autograd.Function):
    """(x, f, gamma, beta, eps) -> (xsum, y) with xsum = x + f and y = LayerNorm(xsum): a pre-LN
    block's residual add and the LayerNorm after it (gpt/gpt.py:147-150) in one pass each way.
    The backward gets the gradient of xsum from its next use (the next residual add) and of y
    from the sublayer, and returns their sum, LayerNorm backward included, for x and f alike:
    the same bits as ``x + f`` then ``CudaLayerNorm`` with autograd summing the two paths, but
    one kernel instead of two in each direction and no separate accumulation."""

    @staticmethod
    def forward(ctx, x, f, gamma, beta, eps=1e-5):
        xsum, y, mean, rstd = add_layernorm_fwd(x, f, gamma, beta, eps)
        ctx.save_for_backward(xsum, gamma, mean, rstd)
        ctx.set_materialize_grads(False)
        return xsum, y

    @staticmethod
    def backward(ctx, grad_xsum, grad_y):
        xsum, gamma, mean, rstd = ctx.saved_tensors
        if grad_y is None:
            return grad_xsum, grad_xsum, None, None, None
        if grad_xsum is None:
            dx, dgamma, dbeta = layernorm_bwd(xsum, gamma, mean, rstd, grad_y.contiguous())
        else:
            dx, dgamma, dbeta = add_layernorm_bwd(xsum, gamma, mean, rstd, grad_y.contiguous(),
                                                  grad_xsum.contiguous())
        return dx, dx, dgamma.reshape(gamma.shape), dbeta.reshape(gamma.shape), None


class CudaLayerNorm(torch.autograd.Function):
    """LayerNorm over the last dim: (x, gamma, beta, eps) -> y (semantics of gpt.py:47-59)."""

    @staticmethod
    def forward(ctx, x, gamma, beta, eps=1e-5):
        y, mean, rstd = layernorm_fwd(x, gamma, beta, eps)
        ctx.save_for_backward(x, gamma, mean, rstd)
        return y

    @staticmethod
    def backward(ctx, grad_output):
        x, gamma, mean, rstd = ctx.saved_tensors
        dx, dgamma, dbeta = layernorm_bwd(x, gamma, mean, rstd, grad_output.contiguous())
        return dx, dgamma.reshape(gamma.shape), dbeta.reshape(gamma.shape), None


class CudaEmbedding(torch.autograd.Function):
    """(tokens, wte, wpe) -> wte[tokens] + wpe[:T], the GPT's token + position embedding
    (gpt/gpt.py:61-72), with a backward that issues no device-to-host read.

    torch's embedding backward sorts the token ids and reads the number of distinct ids back
    to the host.  At the end of a training step's backward that read drains the stream, and
    the GPU then idles while the host issues the optimizer and the next forward (about 0.45 ms
    of a 10.5 ms small-GPT step).  Here the token table's gradient is one GEMM on cuda_fma,
    onehot(tokens)^T . dy, summed in a fixed order (deterministic), when the one-hot matrix is
    small and cheap (vocab x tokens <= ONEHOT_LIMIT floats and 2 vocab tokens width <=
    ONEHOT_FLOP_LIMIT: about 40 us of GEMM, well under the stall it removes); larger vocabularies
    take torch's embedding backward.  The position table's gradient is dy summed over the batch (zero rows past T).
    """

    ONEHOT_LIMIT = 1 << 26
    ONEHOT_FLOP_LIMIT = 4e9

    @staticmethod
    def forward(ctx, tokens, wte, wpe):
        ctx.save_for_backward(tokens)
        ctx.rows = (wte.shape[0], wpe.shape[0])
        return F.embedding(tokens, wte) + wpe[: tokens.shape[-1]]

    @staticmethod
    def backward(ctx, grad_output):
        (tokens,) = ctx.saved_tensors
        V, P = ctx.rows
        T, C = tokens.shape[-1], grad_output.shape[-1]
        dy = grad_output.reshape(-1, C).contiguous()
        ids = tokens.reshape(-1).to(torch.int64)  # int32 ids too, as nn.Embedding takes
        dwte = dwpe = None
        if ctx.needs_input_grad[1]:
            if (V * ids.numel() <= CudaEmbedding.ONEHOT_LIMIT
                    and 2.0 * V * ids.numel() * C <= CudaEmbedding.ONEHOT_FLOP_LIMIT):
                onehot = torch.zeros(V, ids.numel(), dtype=dy.dtype, device=dy.device)
                onehot.scatter_(0, ids.view(1, -1), 1.0)
                dwte = cuda_fma(onehot.unsqueeze(0), dy, _zeros(C, dy)).view(V, C)
            else:
                dwte = torch.ops.aten.embedding_dense_backward(dy, ids, V, -1, False)
        if ctx.needs_input_grad[2]:
            dwpe = grad_output.reshape(-1, T, C).sum(0)
            if T < P:
                dwpe = F.pad(dwpe, (0, 0, 0, P - T))
        return None, dwte, dwpe
