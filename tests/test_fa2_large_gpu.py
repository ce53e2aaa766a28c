"""FlashAttention-2 at tensor sizes past 2^31 elements (the "maximum sizes" edge case).

Q, K, V, dO of shape (1, 262151, 64, 128): 2,147,540,992 elements each, just past 2^31, so
every element offset of the last heads overflows a 32-bit index.  The forward and the
stored-dS backward run on the whole tensors (about 73 GB of FP32 buffers on the 288 GB MI355X);
the first, middle and last heads are checked against the float64 oracle at the tolerances of the
other FA2 tests.  Inputs are generated on the GPU from a fixed seed.

The FP32 dS workspace of all 262151 heads is 3.0 GiB causal and 4.0 GiB non-causal, under the
operator's 8 GiB cap, so the backward runs in one chunk here; the head-chunked schedule is
checked at full size by test_fa2_config3_gpu.py (N = 8192 and 16384: 4 and 16 chunks).
"""
import numpy as np
import pytest
import torch

from conftest import assert_rel_err
from oracle import attention as ora

pytestmark = pytest.mark.gpu

NH, T, HS = 262151, 64, 128
HEADS = [0, 1, NH // 2, NH - 2, NH - 1]


def _gpu_inputs(cuda, dtype, seed):
    g = torch.Generator(device=cuda).manual_seed(seed)
    out = []
    for kind in ("randn", "randn", "randn", "rand"):
        fn = torch.randn if kind == "randn" else torch.rand
        out.append(fn((1, NH, T, HS), generator=g, device=cuda, dtype=torch.float32).to(dtype))
    return out


def _heads(t):
    return t[:, HEADS].detach().double().cpu().numpy()


def _free():
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("causal", [True, False])
def test_fa2_fp32_past_2_to_31_elements(cuda, causal):
    from cuda_transformer.ops import flash_attention_bwd, flash_attention_fwd

    assert NH * T * HS > 2**31
    q, k, v, do = _gpu_inputs(cuda, torch.float32, seed=31 + int(causal))
    O, L = flash_attention_fwd(q, k, v, causal)
    dq, dk, dv = flash_attention_bwd(q, k, v, O, do, L, causal)
    qh, kh, vh, doh = (_heads(t) for t in (q, k, v, do))
    Oh, Lh, dqh, dkh, dvh = (_heads(t) for t in (O, L, dq, dk, dv))
    del q, k, v, do, O, L, dq, dk, dv
    _free()

    O_ref, L_ref = ora.reference_attention(qh, kh, vh, causal)
    np.testing.assert_allclose(Oh, O_ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(Lh, L_ref, rtol=1e-5, atol=1e-5)
    # the kernels' backward used the kernels' own O and L, as the reference's test feeds O
    refs = ora.fa2_backward(qh, kh, vh, Oh, doh, Lh, causal, br=64, bc=64)
    for got, ref in zip((dqh, dkh, dvh), refs):
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-4)
        assert_rel_err(got, ref, 1e-3)


def test_fa2_bf16_past_2_to_31_elements(cuda):
    from cuda_transformer.ops import flash_attention_bwd, flash_attention_fwd

    q, k, v, do = _gpu_inputs(cuda, torch.bfloat16, seed=37)
    O, L = flash_attention_fwd(q, k, v, True)
    dq, dk, dv = flash_attention_bwd(q, k, v, O, do, L, True)
    qh, kh, vh, doh = (_heads(t) for t in (q, k, v, do))
    Oh, Lh, dqh, dkh, dvh = (_heads(t) for t in (O, L, dq, dk, dv))
    del q, k, v, do, O, L, dq, dk, dv
    _free()

    # float64 oracle on the bfloat16-rounded inputs, at the bounds of the other 16-bit tests
    O_ref, L_ref = ora.reference_attention(qh, kh, vh, True)
    bound = 2.0**-8 * (np.abs(O_ref) + np.abs(vh).max(axis=(2, 3), keepdims=True))
    assert np.all(np.abs(Oh - O_ref) <= bound)
    np.testing.assert_allclose(Lh, L_ref, rtol=0, atol=1e-4)
    refs = ora.fa2_backward(qh, kh, vh, O_ref, doh, L_ref, True, br=64, bc=64)
    for got, ref, tol in zip((dqh, dkh, dvh), refs, (3e-2, 3e-2, 1.5e-2)):
        assert_rel_err(got, ref, tol)
