"""Small GPT on the gfx950 kernels: the training-step harness of benchmark config 5.

A parametrised counterpart of the reference's gpt/gpt.py:47-187, whose model reads module
globals (d_model, vocab_size, block_size: gpt.py:17-29,50-51,64-65) and trains at import time.
Same architecture and parameter layout: token + position embedding, pre-LN decoder blocks
(x + attn(ln1(x)), x + mlp(ln2(x)); gpt.py:147-150), fused qkv projection with weights stored
(d_model, 3*d_model) as the reference's `cuda_fma` expects (gpt.py:82-88), causal
FlashAttention-2 on head views of the packed qkv (gpt.py:104-109), MLP 4x with exact GELU
(gpt.py:121-137), final LayerNorm and lm_head, cross-entropy (gpt.py:166-175).  Every linear,
attention, GELU and LayerNorm op runs on the HIP kernels through the reference's autograd
API; the embedding lookups and the cross-entropy stay in torch, as in the reference, while the
token table's gradient is a GEMM on the HIP kernels (CudaEmbedding).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from .autograd_fns import (CudaAddLayerNorm, CudaEmbedding, CudaFlashAttention, CudaFlashAttentionQKV,
                           CudaGeluLayer, CudaLayerNorm, CudaLinearLayer, CudaMLP)


@dataclass
class GPTConfig:
    vocab_size: int = 65
    d_model: int = 384
    n_heads: int = 6
    n_layers: int = 6
    block_size: int = 256
    mlp_ratio: int = 4
    eps: float = 1e-5
    init_std: float = 0.02
    # MLP as one CudaMLP (GELU folded into the fc1 forward and fc2 dx GEMM epilogues; same
    # bits) instead of the reference's CudaLinearLayer -> CudaGeluLayer -> CudaLinearLayer.
    fused_mlp: bool = True
    # Attention on the packed qkv projection (CudaFlashAttentionQKV: O and the qkv gradient
    # written in the packed layouts) instead of the reference's head views, transposes and
    # concatenation around CudaFlashAttention; same kernels, same bits.
    packed_attention: bool = True
    # Each residual add fused with the LayerNorm that follows it (CudaAddLayerNorm: x + f and
    # LayerNorm(x + f) in one pass; in the backward the residual gradient joins the LayerNorm
    # gradient in the same pass) instead of separate adds; same bits.
    fused_residual_ln: bool = True
    # Token + position embedding through CudaEmbedding, whose backward issues no device-to-host
    # read (torch's embedding backward reads the distinct-id count back and stalls the step);
    # the token table's gradient is then summed in another order than torch's.
    cuda_embedding: bool = True


class LayerNorm(nn.Module):
    """LayerNorm over the last dim with the reference's parameter names (gpt.py:47-59)."""

    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.alpha = nn.Parameter(torch.ones(cfg.d_model))
        self.beta = nn.Parameter(torch.zeros(cfg.d_model))
        self.epsilon = cfg.eps

    def forward(self, x):
        return CudaLayerNorm.apply(x, self.alpha, self.beta, self.epsilon)


class Embedding(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.embedding = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.positional = nn.Embedding(cfg.block_size, cfg.d_model)
        self.cuda_embedding = cfg.cuda_embedding

    def forward(self, tokens):
        if self.cuda_embedding:
            return CudaEmbedding.apply(tokens, self.embedding.weight, self.positional.weight)
        T = tokens.shape[1]
        return self.embedding(tokens) + self.positional(torch.arange(T, device=tokens.device))


class CausalSelfAttention(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        d = cfg.d_model
        self.num_heads = cfg.n_heads
        self.head_dim = d // cfg.n_heads
        self.qkv_weight = nn.Parameter(torch.empty(d, 3 * d))
        self.qkv_bias = nn.Parameter(torch.zeros(3 * d))
        self.out_weight = nn.Parameter(torch.empty(d, d))
        self.out_bias = nn.Parameter(torch.zeros(d))
        nn.init.normal_(self.qkv_weight, mean=0.0, std=cfg.init_std)
        nn.init.normal_(self.out_weight, mean=0.0, std=cfg.init_std)
        self.packed = cfg.packed_attention

    def forward(self, x):
        B, T, C = x.shape
        qkv = CudaLinearLayer.apply(x, self.qkv_weight, self.qkv_bias)
        if self.packed:
            # heads read from and written to the packed layouts in place
            att = CudaFlashAttentionQKV.apply(qkv, self.num_heads, True)
        else:
            q, k, v = (t.reshape(B, T, self.num_heads, self.head_dim).transpose(1, 2)
                       for t in qkv.chunk(3, dim=-1))
            att, _ = CudaFlashAttention.apply(q, k, v, True)
            att = att.transpose(1, 2).reshape(B, T, C)
        return CudaLinearLayer.apply(att, self.out_weight, self.out_bias)


class MLP(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        d, h = cfg.d_model, cfg.mlp_ratio * cfg.d_model
        self.fc1_weights = nn.Parameter(torch.empty(d, h))
        self.fc1_bias = nn.Parameter(torch.zeros(h))
        self.fc2_weights = nn.Parameter(torch.empty(h, d))
        self.fc2_bias = nn.Parameter(torch.zeros(d))
        nn.init.normal_(self.fc1_weights, mean=0.0, std=cfg.init_std)
        nn.init.normal_(self.fc2_weights, mean=0.0, std=cfg.init_std)
        self.fused = cfg.fused_mlp

    def forward(self, x):
        if self.fused:
            return CudaMLP.apply(x, self.fc1_weights, self.fc1_bias, self.fc2_weights,
                                 self.fc2_bias)
        x = CudaLinearLayer.apply(x, self.fc1_weights, self.fc1_bias)
        x = CudaGeluLayer.apply(x)
        return CudaLinearLayer.apply(x, self.fc2_weights, self.fc2_bias)


class DecoderBlock(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.ln1 = LayerNorm(cfg)
        self.attn = CausalSelfAttention(cfg)
        self.ln2 = LayerNorm(cfg)
        self.mlp = MLP(cfg)

    def forward(self, x):
        x = x + self.attn(self.ln1(x))
        return x + self.mlp(self.ln2(x))


class GPT(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.cfg = cfg
        self.embedding = Embedding(cfg)
        self.mha = nn.ModuleList([DecoderBlock(cfg) for _ in range(cfg.n_layers)])
        self.ln = LayerNorm(cfg)
        self.lm_head_weights = nn.Parameter(torch.empty(cfg.d_model, cfg.vocab_size))
        self.lm_head_bias = nn.Parameter(torch.zeros(cfg.vocab_size))
        nn.init.normal_(self.lm_head_weights, mean=0.0, std=cfg.init_std)

    def forward(self, idx, targets=None):
        x = self.embedding(idx)
        if self.cfg.fused_residual_ln and len(self.mha) > 0:
            # the blocks' x + attn(ln1(x)), x + mlp(ln2(x)) with every add fused with the next
            # LayerNorm: ln2 of the block, then ln1 of the next block or the final LayerNorm
            z = self.mha[0].ln1(x)
            for i, block in enumerate(self.mha):
                x, z = _add_ln(x, block.attn(z), block.ln2)
                nxt = self.mha[i + 1].ln1 if i + 1 < len(self.mha) else self.ln
                x, z = _add_ln(x, block.mlp(z), nxt)
        else:
            for block in self.mha:
                x = block(x)
            z = self.ln(x)
        logits = CudaLinearLayer.apply(z, self.lm_head_weights, self.lm_head_bias)
        loss = None
        if targets is not None:
            B, T, V = logits.shape
            loss = F.cross_entropy(logits.reshape(B * T, V), targets.reshape(B * T))
        return logits, loss


def _add_ln(x, f, ln: LayerNorm):
    """(x + f, ln(x + f)) through one CudaAddLayerNorm."""
    return CudaAddLayerNorm.apply(x, f, ln.alpha, ln.beta, ln.epsilon)


def init_weights_(model: nn.Module, seed: int, std: float = 0.02) -> None:
    """Deterministic N(0, std^2) init of every weight matrix and embedding, zero biases, unit
    LayerNorm scales — drawn on the CPU so a CPU model initialised the same way matches."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("alpha"):
                p.fill_(1.0)
            elif name.endswith(("beta", "bias")):
                p.zero_()
            else:
                p.copy_(torch.randn(p.shape, generator=g) * std)


def synthetic_batch(cfg: GPTConfig, batch: int, seed: int, device="cpu"):
    """Token ids ~ U[0, vocab) from a seed; targets are the inputs shifted by one."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, cfg.vocab_size, (batch, cfg.block_size + 1), generator=g)
    return ids[:, :-1].to(device), ids[:, 1:].to(device)
