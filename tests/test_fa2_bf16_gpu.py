"""FlashAttention-2 forward with bfloat16 Q, K, V on the GPU vs the CPU oracle (float64).

The oracle is evaluated on the bf16-rounded inputs, so input rounding is not counted as kernel
error.  The kernel accumulates in FP32 and rounds twice: the probabilities to bf16 as the P.V
operand, and O to bf16 on output, each a relative error of at most 2^-9.  Hence per element
    |O - O_ref| <= 2^-9 |O_ref| + 2^-9 max_j |v_j| (+ FP32 accumulation),
bounded here by 2^-8 (|O_ref| + max|V|); L comes from FP32 scores of exact bf16 products and
keeps an FP32-level bound of 1e-4.  Shapes follow the FP32 suite (ragged T, causal and full,
hs 64 and 128, benchmark config 1).
"""
import numpy as np
import pytest
import torch

from conftest import f64, seeded
from oracle import attention as ora

pytestmark = pytest.mark.gpu

SHAPES = [
    (1, 4, 256, 64, True),   # benchmark config 1
    (1, 4, 256, 64, False),  # benchmark config 1
    (1, 1, 65, 64, True),
    (2, 4, 128, 64, True),
    (2, 4, 257, 64, True),
    (1, 2, 200, 128, False),
    (1, 2, 512, 128, True),
    (1, 3, 1, 64, True),     # single row
    (2, 2, 1000, 64, False),
    (1, 2, 1030, 128, True),
]


def _bf16_inputs(B, nh, T, hs, seed):
    return [seeded((B, nh, T, hs), seed + i).to(torch.bfloat16) for i in range(3)]


def _check(O, L, q, k, v, causal):
    O_ref, L_ref = ora.reference_attention(f64(q), f64(k), f64(v), causal)
    assert O.dtype == torch.bfloat16 and L.dtype == torch.float32
    bound = 2.0 ** -8 * (np.abs(O_ref) + np.abs(f64(v)).max())
    err = np.abs(f64(O) - O_ref)
    assert (err <= bound).all(), f"O error {err.max():.3e} exceeds the bf16 bound"
    assert np.abs(f64(L) - L_ref).max() <= 1e-4
    return err.max()


@pytest.mark.parametrize("B,nh,T,hs,causal", SHAPES)
def test_fa2_bf16_forward_matches_oracle(cuda, B, nh, T, hs, causal):
    from cuda_transformer.ops import flash_attention_fwd

    q, k, v = _bf16_inputs(B, nh, T, hs, seed=3000 + T + hs)
    O, L = flash_attention_fwd(q.to(cuda), k.to(cuda), v.to(cuda), causal)
    torch.cuda.synchronize()
    _check(O.cpu(), L.cpu(), q, k, v, causal)


def test_fa2_bf16_forward_error_like_torch_bf16(cuda):
    """The kernel's error against the float64 oracle is no larger than that of torch's own
    bf16 attention (CPU SDPA on the same bf16 inputs) plus the bf16 output rounding."""
    import torch.nn.functional as F

    from cuda_transformer.ops import flash_attention_fwd

    q, k, v = _bf16_inputs(1, 4, 256, 64, seed=77)
    O, _ = flash_attention_fwd(q.to(cuda), k.to(cuda), v.to(cuda), True)
    O_ref, _ = ora.reference_attention(f64(q), f64(k), f64(v), True)
    ours = np.abs(f64(O) - O_ref).mean()
    torch_bf16 = np.abs(f64(F.scaled_dot_product_attention(q, k, v, is_causal=True)) - O_ref).mean()
    assert ours <= 1.5 * torch_bf16 + 1e-4, (ours, torch_bf16)


def test_fa2_bf16_strided_views(cuda):
    """Head views of a packed (B, T, 3C) bf16 projection are read in place, as in gpt.py."""
    from cuda_transformer.ops import flash_attention_fwd

    B, T, nh, hs = 2, 96, 3, 64
    qkv = seeded((B, T, 3 * nh * hs), 5).to(torch.bfloat16)
    q, k, v = (t.view(B, T, nh, hs).transpose(1, 2) for t in qkv.split(nh * hs, dim=2))
    g = qkv.to(cuda)
    qg, kg, vg = (t.view(B, T, nh, hs).transpose(1, 2) for t in g.split(nh * hs, dim=2))
    O, L = flash_attention_fwd(qg, kg, vg, True)
    torch.cuda.synchronize()
    _check(O.cpu(), L.cpu(), q.contiguous(), k.contiguous(), v.contiguous(), True)


def test_fa2_bf16_deterministic(cuda):
    from cuda_transformer.ops import flash_attention_fwd

    q, k, v = (t.to(cuda) for t in _bf16_inputs(2, 4, 300, 128, seed=11))
    O1, L1 = flash_attention_fwd(q, k, v, True)
    O2, L2 = flash_attention_fwd(q, k, v, True)
    assert torch.equal(O1, O2) and torch.equal(L1, L2)


def test_fa2_bf16_errors(cuda):
    from cuda_transformer.ops import flash_attention_fwd

    q = torch.randn(1, 2, 16, 32, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="hs=64 and hs=128"):
        flash_attention_fwd(q, q, q, False)
    q = torch.randn(1, 2, 16, 64, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="all be bfloat16"):
        flash_attention_fwd(q, q.float(), q, False)
