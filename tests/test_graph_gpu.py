"""The operators under HIP graph capture (torch.cuda.CUDAGraph on ROCm records a hipGraph).

Every op allocates through torch and launches on the current stream with no host
synchronisation, no hipMalloc and no memset node, so a training step built from them can be
captured once and replayed without launch overhead.  The test captures FlashAttention-2 forward
+ backward (FP32, and BF16 in both backward schedules), the GEMM (including a split-K shape, whose workspace and reduction
kernel are captured too), bias gradient, GELU (both forms), softmax and LayerNorm forward + backward; then it
replays the graph several times on fresh inputs, with eager work between replays, and requires
every replay to equal the eager result bit for bit.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _fill(tensors, seed):
    g = torch.Generator().manual_seed(seed)
    for t in tensors:
        t.copy_(torch.randn(t.shape, generator=g).to(t.dtype))


def test_ops_replay_in_a_hip_graph(cuda):
    from cuda_transformer.ops import (cuda_fma, cuda_softmax, cuda_softmax_bwd, db_calculation,
                                      flash_attention_bwd, flash_attention_fwd, gelu_activation,
                                      gelu_activation_bwd, gelu_tanh_activation,
                                      gelu_tanh_activation_bwd, layernorm_bwd, layernorm_fwd)

    q, k, v, do = (torch.empty(2, 4, 257, 64, device=cuda) for _ in range(4))
    qh, kh, vh, doh = (torch.empty(1, 2, 200, 128, device=cuda, dtype=torch.bfloat16)
                       for _ in range(4))
    # hs 64: the 16-bit backward's recompute schedule (hs 128 above: the stored one)
    q6, k6, v6, do6 = (torch.empty(2, 3, 130, 64, device=cuda, dtype=torch.bfloat16)
                       for _ in range(4))
    x = torch.empty(2, 96, 384, device=cuda)
    w = torch.empty(384, 512, device=cuda)
    bias = torch.empty(512, device=cuda)
    xs = torch.empty(1, 4096, 128, device=cuda)   # x^T . y with K = 4096: split along K
    ys = torch.empty(1, 4096, 96, device=cuda)
    gamma, beta = torch.empty(384, device=cuda), torch.empty(384, device=cuda)
    inputs = [q, k, v, do, qh, kh, vh, doh, q6, k6, v6, do6, x, w, bias, xs, ys, gamma, beta]

    def step():
        O, L = flash_attention_fwd(q, k, v, True)
        grads = flash_attention_bwd(q, k, v, O, do, L, True)
        Oh, Lh = flash_attention_fwd(qh, kh, vh, False)
        grads_h = flash_attention_bwd(qh, kh, vh, Oh, doh, Lh, False)
        O6, L6 = flash_attention_fwd(q6, k6, v6, True)
        grads_6 = flash_attention_bwd(q6, k6, v6, O6, do6, L6, True)
        y = cuda_fma(x, w, bias)
        yk = cuda_fma(xs.transpose(1, 2), ys, torch.zeros(96, device=cuda))
        gy = gelu_activation(y)
        dgy = gelu_activation_bwd(y, gy)
        ty = gelu_tanh_activation(y)
        dty = gelu_tanh_activation_bwd(y, ty)
        p = cuda_softmax(gy)
        dp = cuda_softmax_bwd(p, gy)
        db = db_calculation(dgy)
        ln, mean, rstd = layernorm_fwd(x, gamma, beta)
        lgrads = layernorm_bwd(x, gamma, mean, rstd, ln)
        return (O, L, *grads, Oh, Lh, *grads_h, O6, L6, *grads_6, y, yk, gy, dgy, ty, dty, p, dp, db, ln, mean,
                rstd, *lgrads)

    _fill(inputs, 0)
    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()

    for rep in range(4):
        _fill(inputs, 100 + rep)
        graph.replay()
        torch.cuda.synchronize()
        eager = step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(captured, eager)):
            assert torch.equal(a, b), f"replay {rep}: output {i} differs from the eager result"
