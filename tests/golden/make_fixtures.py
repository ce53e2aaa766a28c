"""Write the golden fixtures in this directory (run: python tests/golden/make_fixtures.py).

The reference holds no golden vectors (its tests draw unseeded random inputs and compare
against torch on the fly: test/test_flash_attention.py:10-50, test_linear.py:10-51,
test_gelu.py:10-31, test_softmax.py:10-31, test_causal_self_attn.py:10-62).  These fixtures
freeze that same oracle — torch's CPU math in float64, evaluated on float32 inputs drawn from
fixed seeds — so that the numpy oracle and the HIP kernels are both checked against values
that neither of them produced.  Inputs are stored as float32 (the kernels' type), expected
outputs as float64.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

HERE = Path(__file__).resolve().parent


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _randn(shape, seed, scale=1.0):
    return torch.randn(shape, generator=_gen(seed), dtype=torch.float32) * scale


def _rand(shape, seed):
    return torch.rand(shape, generator=_gen(seed), dtype=torch.float32)


def fa2_case(name, B, nh, T, hs, causal, seed):
    q, k, v = (_randn((B, nh, T, hs), seed + i) for i in range(3))
    do = _rand((B, nh, T, hs), seed + 3)
    q64, k64, v64 = (t.double().requires_grad_() for t in (q, k, v))
    scale = hs ** -0.5
    with sdpa_kernel(SDPBackend.MATH):
        o = F.scaled_dot_product_attention(q64, k64, v64, is_causal=causal, scale=scale)
    s = (q64 @ k64.transpose(-2, -1)) * scale
    if causal:
        s = s.masked_fill(torch.tril(torch.ones(T, T, dtype=torch.bool)) == 0, float("-inf"))
    L = torch.logsumexp(s, dim=-1)
    dq, dk, dv = torch.autograd.grad(o, (q64, k64, v64), grad_outputs=do.double())
    np.savez_compressed(HERE / f"{name}.npz", q=q.numpy(), k=k.numpy(), v=v.numpy(),
                        do=do.numpy(), causal=np.array(causal), o=o.detach().numpy(),
                        L=L.detach().numpy(), dq=dq.numpy(), dk=dk.numpy(), dv=dv.numpy())


def linear_case(name, B, T, fin, fout, seed):
    x = _rand((B, T, fin), seed)
    w = _randn((fin, fout), seed + 1, 0.1)
    b = _randn((fout,), seed + 2, 0.1)
    dy = _rand((B, T, fout), seed + 3)
    x64, w64, b64 = (t.double().requires_grad_() for t in (x, w, b))
    out = x64 @ w64 + b64
    dx, dw, db = torch.autograd.grad(out, (x64, w64, b64), grad_outputs=dy.double())
    np.savez_compressed(HERE / f"{name}.npz", x=x.numpy(), w=w.numpy(), b=b.numpy(),
                        dy=dy.numpy(), out=out.detach().numpy(), dx=dx.numpy(), dw=dw.numpy(),
                        db=db.numpy())


def gelu_case(name, shape, seed):
    x = _rand(shape, seed) * 8 - 4
    dy = _rand(shape, seed + 1)
    x64 = x.double().requires_grad_()
    y = F.gelu(x64)  # default: exact erf form, as test_gelu.py:16 uses
    (dx,) = torch.autograd.grad(y, (x64,), grad_outputs=dy.double())
    np.savez_compressed(HERE / f"{name}.npz", x=x.numpy(), dy=dy.numpy(),
                        y=y.detach().numpy(), dx=dx.numpy())


def softmax_case(name, shape, seed, scale):
    x = _randn(shape, seed, scale)
    dp = _rand(shape, seed + 1)
    x64 = x.double().requires_grad_()
    p = F.softmax(x64, dim=-1)
    (dx,) = torch.autograd.grad(p, (x64,), grad_outputs=dp.double())
    np.savez_compressed(HERE / f"{name}.npz", x=x.numpy(), dp=dp.numpy(), p=p.detach().numpy(),
                        dx=dx.numpy())


def layernorm_case(name, rows, n, seed):
    x = _randn((rows, n), seed, 2.0) + 0.5
    g = 1 + _randn((n,), seed + 1, 0.1)
    b = _randn((n,), seed + 2, 0.1)
    dy = _randn((rows, n), seed + 3)
    x64, g64, b64 = (t.double().requires_grad_() for t in (x, g, b))
    y = F.layer_norm(x64, (n,), g64, b64, eps=1e-5)
    dx, dg, db = torch.autograd.grad(y, (x64, g64, b64), grad_outputs=dy.double())
    np.savez_compressed(HERE / f"{name}.npz", x=x.numpy(), gamma=g.numpy(), beta=b.numpy(),
                        dy=dy.numpy(), y=y.detach().numpy(), dx=dx.numpy(), dgamma=dg.numpy(),
                        dbeta=db.numpy())


def naive_attention_case(name, B, T, nh, hs, causal, seed):
    C = nh * hs
    qkv = _rand((B, T, 3 * C), seed)
    dO = _rand((B, T, C), seed + 1)
    x = qkv.double().requires_grad_()
    q, k, v = x[..., :C], x[..., C:2 * C], x[..., 2 * C:]
    q, k, v = (t.reshape(B, T, nh, hs).transpose(1, 2) for t in (q, k, v))
    s = (q @ k.transpose(-2, -1)) * hs ** -0.5
    if causal:
        s = s.masked_fill(torch.tril(torch.ones(T, T, dtype=torch.bool)) == 0, float("-inf"))
    p = F.softmax(s, dim=-1)
    out = (p @ v).transpose(1, 2).reshape(B, T, C)
    (dqkv,) = torch.autograd.grad(out, (x,), grad_outputs=dO.double())
    np.savez_compressed(HERE / f"{name}.npz", qkv=qkv.numpy(), dO=dO.numpy(), nh=np.array(nh),
                        causal=np.array(causal), out=out.detach().numpy(),
                        probs=p.detach().numpy(), dqkv=dqkv.numpy())


def main():
    torch.set_num_threads(4)
    fa2_case("fa2_b1h1t65d64_causal", 1, 1, 65, 64, True, 100)
    fa2_case("fa2_b1h2t33d32_full", 1, 2, 33, 32, False, 200)
    fa2_case("fa2_b1h1t17d128_causal", 1, 1, 17, 128, True, 300)
    fa2_case("fa2_b2h1t24d64_full", 2, 1, 24, 64, False, 400)
    linear_case("linear_b1t32i65o32", 1, 32, 65, 32, 500)
    linear_case("linear_b2t20i33o48", 2, 20, 33, 48, 510)
    gelu_case("gelu_1x65x32", (1, 65, 32), 600)
    softmax_case("softmax_2x9x70", (2, 9, 70), 700, 2.0)
    softmax_case("softmax_1x4x1024", (1, 4, 1024), 710, 2.0)
    layernorm_case("layernorm_9x768", 9, 768, 800)
    layernorm_case("layernorm_5x65", 5, 65, 810)
    naive_attention_case("naive_b1t33h2d32_causal", 1, 33, 2, 32, True, 900)
    naive_attention_case("naive_b2t17h1d64_full", 2, 17, 1, 64, False, 910)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
