"""The GPT harness on the CPU: the kernel model and the plain-torch oracle model have the same
parameters (so a state dict copies across), and the oracle model's pieces match torch's own."""
import math

import torch
import torch.nn.functional as F

from cuda_transformer_amd.gpt import GPT, GPTConfig, init_weights_, synthetic_batch
from oracle import gpt as ogpt


def test_parameter_layout_matches_oracle():
    cfg = GPTConfig(n_layers=2)
    a, b = GPT(cfg), ogpt.GPT(cfg)
    sa = {k: v.shape for k, v in a.state_dict().items()}
    sb = {k: v.shape for k, v in b.state_dict().items()}
    assert sa == sb
    n = sum(p.numel() for p in GPT(GPTConfig()).parameters())
    assert 10_700_000 < n < 10_900_000  # the 10.8 M-parameter config 5 model


def test_oracle_model_initial_loss_and_attention():
    cfg = GPTConfig(n_layers=2, block_size=32)
    m = ogpt.GPT(cfg)
    init_weights_(m, seed=0)
    idx, tgt = synthetic_batch(cfg, 4, seed=1)
    _, loss = m(idx, tgt)
    # the final LayerNorm gives unit-variance features, so logits ~ N(0, d * std^2) and the
    # expected loss is ln(vocab) + d * std^2 / 2
    expect = math.log(cfg.vocab_size) + cfg.d_model * cfg.init_std ** 2 / 2
    assert abs(loss.item() - expect) < 0.03
    # attention block == torch SDPA causal on the same projections
    attn = m.mha[0].attn
    x = torch.randn(2, 32, cfg.d_model)
    qkv = x @ attn.qkv_weight + attn.qkv_bias
    q, k, v = (t.reshape(2, 32, cfg.n_heads, 64).transpose(1, 2) for t in qkv.chunk(3, -1))
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True).transpose(1, 2).reshape(2, 32, -1)
    torch.testing.assert_close(attn(x), ref @ attn.out_weight + attn.out_bias, rtol=1e-5, atol=1e-5)
    # LayerNorm restatement == F.layer_norm
    ln = m.ln
    torch.testing.assert_close(ln(x), F.layer_norm(x, (cfg.d_model,), ln.alpha, ln.beta, 1e-5),
                               rtol=1e-5, atol=1e-5)
