"""Plain-torch restatement of the reference's GPT (gpt/gpt.py:47-187) — TEST INFRASTRUCTURE ONLY.

The CPU reference for the training-step harness: the same modules and parameter names as
cuda_transformer_amd.gpt, computed with torch math on the CPU (LayerNorm as gpt.py:54-59,
linear as x @ W + b with W stored (in, out), causal softmax attention with scale 1/sqrt(hs),
exact GELU).  A state dict copies across unchanged, so both models start from identical
weights and see identical token ids.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F


class LayerNorm(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.alpha = nn.Parameter(torch.ones(cfg.d_model))
        self.beta = nn.Parameter(torch.zeros(cfg.d_model))
        self.epsilon = cfg.eps

    def forward(self, x):  # gpt.py:54-59
        var = torch.var(x, dim=-1, keepdim=True, unbiased=False)
        mean = torch.mean(x, dim=-1, keepdim=True)
        return (x - mean) / torch.sqrt(var + self.epsilon) * self.alpha + self.beta


class Embedding(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.embedding = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.positional = nn.Embedding(cfg.block_size, cfg.d_model)

    def forward(self, tokens):
        T = tokens.shape[1]
        return self.embedding(tokens) + self.positional(torch.arange(T, device=tokens.device))


class CausalSelfAttention(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        d = cfg.d_model
        self.num_heads = cfg.n_heads
        self.head_dim = d // cfg.n_heads
        self.qkv_weight = nn.Parameter(torch.empty(d, 3 * d))
        self.qkv_bias = nn.Parameter(torch.zeros(3 * d))
        self.out_weight = nn.Parameter(torch.empty(d, d))
        self.out_bias = nn.Parameter(torch.zeros(d))

    def forward(self, x):
        B, T, C = x.shape
        qkv = x @ self.qkv_weight + self.qkv_bias
        q, k, v = (t.reshape(B, T, self.num_heads, self.head_dim).transpose(1, 2)
                   for t in qkv.chunk(3, dim=-1))
        s = (q @ k.transpose(-2, -1)) / math.sqrt(self.head_dim)
        s = s.masked_fill(torch.ones(T, T, dtype=torch.bool).triu(1), float("-inf"))
        att = (F.softmax(s, dim=-1) @ v).transpose(1, 2).reshape(B, T, C)
        return att @ self.out_weight + self.out_bias


class MLP(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        d, h = cfg.d_model, cfg.mlp_ratio * cfg.d_model
        self.fc1_weights = nn.Parameter(torch.empty(d, h))
        self.fc1_bias = nn.Parameter(torch.zeros(h))
        self.fc2_weights = nn.Parameter(torch.empty(h, d))
        self.fc2_bias = nn.Parameter(torch.zeros(d))

    def forward(self, x):
        return F.gelu(x @ self.fc1_weights + self.fc1_bias) @ self.fc2_weights + self.fc2_bias


class DecoderBlock(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.ln1 = LayerNorm(cfg)
        self.attn = CausalSelfAttention(cfg)
        self.ln2 = LayerNorm(cfg)
        self.mlp = MLP(cfg)

    def forward(self, x):
        x = x + self.attn(self.ln1(x))
        return x + self.mlp(self.ln2(x))


class GPT(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.cfg = cfg
        self.embedding = Embedding(cfg)
        self.mha = nn.ModuleList([DecoderBlock(cfg) for _ in range(cfg.n_layers)])
        self.ln = LayerNorm(cfg)
        self.lm_head_weights = nn.Parameter(torch.empty(cfg.d_model, cfg.vocab_size))
        self.lm_head_bias = nn.Parameter(torch.zeros(cfg.vocab_size))

    def forward(self, idx, targets=None):
        x = self.embedding(idx)
        for block in self.mha:
            x = block(x)
        logits = self.ln(x) @ self.lm_head_weights + self.lm_head_bias
        loss = None
        if targets is not None:
            B, T, V = logits.shape
            loss = F.cross_entropy(logits.reshape(B * T, V), targets.reshape(B * T))
        return logits, loss
