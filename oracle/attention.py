"""Attention oracle: FlashAttention-2 forward/backward and the materialised attention.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Blocked numpy restatements of the
reference kernels.  Arrays are (B, nh, T, hs); computation runs in the dtype of the inputs
(float64 for checking, float32 for the CPU baseline timing).
"""
from __future__ import annotations

import numpy as np


def softmax_scale(hs: int) -> float:
    """1/sqrt(hs): the launcher passes sqrt(hs) and the kernel inverts it
    (Transformer_launchers/flash_attn_launcher.cu:27, Transformer_kernels/flash_attention.cuh:45)."""
    return 1.0 / np.sqrt(hs)


def _mask(i0: int, i1: int, j0: int, j1: int, causal: bool) -> np.ndarray | None:
    """True where a score is masked: j > i when causal (flash_attention.cuh:117,:304,:446)."""
    if not causal:
        return None
    i = np.arange(i0, i1)[:, None]
    j = np.arange(j0, j1)[None, :]
    return j > i


def fa2_forward(q, k, v, causal: bool, br: int = 16, bc: int = 16):
    """Online-softmax forward over K/V tiles, returning (O, L).

    Follows flash_attention_fwd_kernel (flash_attention.cuh:27-170): per query tile, running
    max m and sum l (:53-59), scores S = scale * q k^T masked to -inf (:113-118), KV loop ending
    at the diagonal tile when causal (:80,:86), m_new = max(m, rowmax S), alpha = e^{m - m_new}
    (:124-126), P = e^{S - m_new} (:130-134), l = alpha l + rowsum P (:139), o = alpha o + P v
    (:144-151); finally O = o / l (:163) and L = m + ln l (:167).
    """
    B, H, T, D = q.shape
    dt = np.result_type(q, k, v)
    scale = dt.type(softmax_scale(D))
    O = np.empty((B, H, T, D), dtype=dt)
    L = np.empty((B, H, T), dtype=dt)
    with np.errstate(invalid="ignore", over="ignore"):
        for i0 in range(0, T, br):
            i1 = min(i0 + br, T)
            qt = q[:, :, i0:i1, :]
            m = np.full((B, H, i1 - i0), -np.inf, dtype=dt)
            l = np.zeros((B, H, i1 - i0), dtype=dt)
            o = np.zeros((B, H, i1 - i0, D), dtype=dt)
            q_end = min(i1, T) if causal else T
            for j0 in range(0, q_end, bc):
                j1 = min(j0 + bc, T)
                s = (qt @ np.swapaxes(k[:, :, j0:j1, :], -1, -2)) * scale
                msk = _mask(i0, i1, j0, j1, causal)
                if msk is not None:
                    s = np.where(msk, -np.inf, s)
                m_new = np.maximum(m, s.max(axis=-1))
                alpha = np.exp(m - m_new)
                p = np.exp(s - m_new[..., None])
                l = alpha * l + p.sum(axis=-1)
                o = o * alpha[..., None] + p @ v[:, :, j0:j1, :]
                m = m_new
            O[:, :, i0:i1, :] = o / l[..., None]
            L[:, :, i0:i1] = m + np.log(l)
    return O, L


def fa2_bwd_delta(o, do):
    """delta_i = sum_d O_id dO_id (flash_attention_bwd_delta, flash_attention.cuh:175-213)."""
    return (o * do).sum(axis=-1)


def fa2_bwd_dq(q, k, v, do, L, delta, causal: bool, br: int = 16, bc: int = 16):
    """dQ per query tile (flash_attention_bwd_dq, flash_attention.cuh:216-354): recompute
    S (:295-306) and P = e^{S - L} (:309-312), dP = dO v^T (:315-322),
    dS = P (dP - delta) (:325-328), dQ += scale dS k (:331-338); KV loop ends at the diagonal."""
    B, H, T, D = q.shape
    dt = np.result_type(q, k, v, do)
    scale = dt.type(softmax_scale(D))
    dq = np.zeros_like(q, dtype=dt)
    with np.errstate(invalid="ignore", over="ignore"):
        for i0 in range(0, T, br):
            i1 = min(i0 + br, T)
            q_end = min(i1, T) if causal else T
            acc = np.zeros((B, H, i1 - i0, D), dtype=dt)
            for j0 in range(0, q_end, bc):
                j1 = min(j0 + bc, T)
                s = (q[:, :, i0:i1] @ np.swapaxes(k[:, :, j0:j1], -1, -2)) * scale
                msk = _mask(i0, i1, j0, j1, causal)
                if msk is not None:
                    s = np.where(msk, -np.inf, s)
                p = np.exp(s - L[:, :, i0:i1, None])
                dp = do[:, :, i0:i1] @ np.swapaxes(v[:, :, j0:j1], -1, -2)
                ds = p * (dp - delta[:, :, i0:i1, None])
                acc += (ds @ k[:, :, j0:j1]) * scale
            dq[:, :, i0:i1] = acc
    return dq


def fa2_bwd_dkdv(q, k, v, do, L, delta, causal: bool, br: int = 16, bc: int = 16):
    """dK, dV per key tile (flash_attention_bwd_dk_dv, flash_attention.cuh:357-504):
    dV += P^T dO (:457-463), dP = dO v^T (:466-472), dS = P (dP - delta) (:475-478),
    dK += scale dS^T q (:481-487).  The reference walks every query tile (:411); query tiles
    that lie wholly before the key tile contribute exactly 0 under the causal mask (P = e^{-inf}),
    so this restatement starts at the first query tile that can see the key tile."""
    B, H, T, D = q.shape
    dt = np.result_type(q, k, v, do)
    scale = dt.type(softmax_scale(D))
    dk = np.zeros_like(k, dtype=dt)
    dv = np.zeros_like(v, dtype=dt)
    with np.errstate(invalid="ignore", over="ignore"):
        for j0 in range(0, T, bc):
            j1 = min(j0 + bc, T)
            kt, vt = k[:, :, j0:j1], v[:, :, j0:j1]
            acc_k = np.zeros((B, H, j1 - j0, D), dtype=dt)
            acc_v = np.zeros((B, H, j1 - j0, D), dtype=dt)
            start = (j0 // br) * br if causal else 0
            for i0 in range(start, T, br):
                i1 = min(i0 + br, T)
                s = (q[:, :, i0:i1] @ np.swapaxes(kt, -1, -2)) * scale
                msk = _mask(i0, i1, j0, j1, causal)
                if msk is not None:
                    s = np.where(msk, -np.inf, s)
                p = np.exp(s - L[:, :, i0:i1, None])
                acc_v += np.swapaxes(p, -1, -2) @ do[:, :, i0:i1]
                dp = do[:, :, i0:i1] @ np.swapaxes(vt, -1, -2)
                ds = p * (dp - delta[:, :, i0:i1, None])
                acc_k += (np.swapaxes(ds, -1, -2) @ q[:, :, i0:i1]) * scale
            dk[:, :, j0:j1] = acc_k
            dv[:, :, j0:j1] = acc_v
    return dk, dv


def fa2_backward(q, k, v, o, do, L, causal: bool, br: int = 16, bc: int = 16):
    """The three-stage backward in launch order (flash_attn_launcher.cu:106-133)."""
    delta = fa2_bwd_delta(o, do)
    dq = fa2_bwd_dq(q, k, v, do, L, delta, causal, br, bc)
    dk, dv = fa2_bwd_dkdv(q, k, v, do, L, delta, causal, br, bc)
    return dq, dk, dv


# ------------------------------------------------------------------ naive attention
def causal_self_attention_forward(qkv, nh: int, causal: bool):
    """Materialised attention over packed qkv (B, T, 3C) -> (out (B,T,C), probs (B,nh,T,T)).

    Stage 1 S = (q k^T) / sqrt(hs), -inf above the diagonal when causal
    (causal_self_attention_fwd.cuh:9-67); row softmax (softmax.cuh:25-106, launched in place
    at causal_self_attn_layer.cu:49-54); stage 3 out = P v into (B, T, C)
    (causal_self_attention_fwd.cuh:69-127)."""
    B, T, C3 = qkv.shape
    C = C3 // 3
    hs = C // nh
    dt = qkv.dtype

    def heads(x):
        return np.ascontiguousarray(x.reshape(B, T, nh, hs).transpose(0, 2, 1, 3))

    q, k, v = heads(qkv[..., :C]), heads(qkv[..., C:2 * C]), heads(qkv[..., 2 * C:])
    s = (q @ np.swapaxes(k, -1, -2)) * dt.type(softmax_scale(hs))
    if causal:
        s = np.where(_mask(0, T, 0, T, True), -np.inf, s)
    from .elementwise import softmax_forward

    p = softmax_forward(s)
    out = (p @ v).transpose(0, 2, 1, 3).reshape(B, T, C)
    return out, p


def causal_self_attention_backward(q, k, v, probs, do):
    """Naive backward on (B*nh, T, hs) (causal_self_attn_layer.cu:70-132): dV = P^T dO,
    dP = dO V^T, dS = softmax_bwd(P, dP), dQ = dS K, dK = dS^T Q — dQ, dK unscaled."""
    from .elementwise import softmax_backward

    dv = np.swapaxes(probs, -1, -2) @ do
    dp = do @ np.swapaxes(v, -1, -2)
    ds = softmax_backward(probs, dp)
    dq = ds @ k
    dk = np.swapaxes(ds, -1, -2) @ q
    return dq, dk, dv


def reference_attention(q, k, v, causal: bool):
    """Direct (non-blocked) formula: O = softmax(scale q k^T + mask) v and L = logsumexp —
    the definitions the reference's test uses (test/test_flash_attention.py:10-21,32)."""
    D = q.shape[-1]
    T = q.shape[-2]
    s = (q @ np.swapaxes(k, -1, -2)) * q.dtype.type(softmax_scale(D))
    if causal:
        s = np.where(_mask(0, T, 0, T, True), -np.inf, s)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(axis=-1, keepdims=True)
    return (e / l) @ v, (m + np.log(l))[..., 0]
