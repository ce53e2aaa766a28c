"""Linear, db, GELU (erf and tanh forms), softmax, LayerNorm and naive attention on the GPU vs
the CPU oracle.

Shapes follow the reference suite (test/test_linear.py:53-59, test_gelu.py:36-42,
test_softmax.py:33-39, test_causal_self_attn.py:69-77) plus benchmark config 4 (GPT-2-small
widths).  Tolerances: the reference's allclose atol 1e-5 (rtol 1e-5) on U[0,1) inputs; for
config 4 the GEMM is checked by relative error (K = 768/3072 FP32 sums).
"""
import numpy as np
import pytest
import torch

from conftest import f64, rel_err, seeded
from oracle import attention as ora
from oracle import elementwise as ew
from oracle import linear as lin

pytestmark = pytest.mark.gpu

LINEAR_SHAPES = [(1, 32, 64, 32), (1, 32, 65, 32), (2, 64, 32, 64), (2, 128, 32, 64),
                 (1, 512, 70, 120), (3, 33, 129, 257)]
ROW_SHAPES = [(1, 64, 32), (1, 65, 32), (2, 32, 64), (4, 128, 64), (1, 70, 120), (2, 5, 1000),
              (1, 3, 2049), (1, 2, 5000), (3, 7, 4096)]


@pytest.mark.parametrize("B,T,fin,fout", LINEAR_SHAPES)
def test_linear_forward_backward(cuda, B, T, fin, fout):
    from cuda_autograd_fns import CudaLinearLayer
    from cuda_transformer.ops import cuda_fma, db_calculation

    x = seeded((B, T, fin), 1, kind="rand")
    w = seeded((fin, fout), 2) * 0.1
    b = seeded((fout,), 3) * 0.1
    dy = seeded((B, T, fout), 4, kind="rand")
    out = cuda_fma(x.to(cuda), w.to(cuda), b.to(cuda))
    np.testing.assert_allclose(f64(out), lin.fma_forward(f64(x), f64(w), f64(b)), atol=1e-5,
                               rtol=1e-5)
    # the reference test's own backward composition (test_linear.py:33-51)
    w3 = w.to(cuda).unsqueeze(0).transpose(1, 2)
    dx = cuda_fma(dy.to(cuda), w3, torch.zeros(fin, device=cuda))
    dw = cuda_fma(dy.to(cuda).transpose(1, 2), x.to(cuda), torch.zeros(fin, device=cuda)).sum(0)
    db = db_calculation(dy.to(cuda))
    dx_r, dw_r, db_r = lin.linear_backward(f64(x), f64(w), f64(dy))
    np.testing.assert_allclose(f64(dx), dx_r, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(f64(dw), dw_r.T, atol=1e-4, rtol=1e-5)
    np.testing.assert_allclose(f64(db), db_r, atol=1e-4, rtol=1e-5)
    # autograd wrapper
    xg = x.to(cuda).requires_grad_()
    wg = w.to(cuda).requires_grad_()
    bg = b.to(cuda).requires_grad_()
    CudaLinearLayer.apply(xg, wg, bg).backward(dy.to(cuda))
    np.testing.assert_allclose(f64(xg.grad), dx_r, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(f64(wg.grad), dw_r, atol=1e-4, rtol=1e-5)
    np.testing.assert_allclose(f64(bg.grad), db_r, atol=1e-4, rtol=1e-5)


def test_linear_batched_weights_and_errors(cuda):
    from cuda_transformer.ops import cuda_fma

    x = seeded((3, 40, 24), 1).to(cuda)
    w = seeded((3, 24, 36), 2).to(cuda)
    b = seeded((36,), 3).to(cuda)
    out = cuda_fma(x, w, b)
    np.testing.assert_allclose(f64(out), lin.fma_forward(f64(x), f64(w), f64(b)), atol=1e-4,
                               rtol=1e-5)
    with pytest.raises(RuntimeError, match="weights.size\\(1\\) must match x.size\\(2\\)"):
        cuda_fma(x, w[:, :20], b)
    with pytest.raises(RuntimeError, match="bias.size\\(0\\) must match weights.size\\(2\\)"):
        cuda_fma(x, w, b[:30])


def test_linear_config4(cuda):
    """X[8192,768] . W[768,3072] + b, X and W ~ N(0, 0.02^2) (benchmark config 4)."""
    from cuda_autograd_fns import CudaLinearLayer

    x = seeded((1, 8192, 768), 40, scale=0.02)
    w = seeded((768, 3072), 41, scale=0.02)
    b = seeded((3072,), 42, scale=0.02)
    dy = seeded((1, 8192, 3072), 43, scale=0.02)
    xg, wg, bg = (t.to(cuda).requires_grad_() for t in (x, w, b))
    out = CudaLinearLayer.apply(xg, wg, bg)
    out.backward(dy.to(cuda))
    ref = lin.fma_forward(f64(x), f64(w), f64(b))
    assert rel_err(f64(out), ref) <= 1e-5
    dx_r, dw_r, db_r = lin.linear_backward(f64(x), f64(w), f64(dy))
    assert rel_err(f64(xg.grad), dx_r) <= 1e-5
    assert rel_err(f64(wg.grad), dw_r) <= 1e-5
    assert rel_err(f64(bg.grad), db_r) <= 1e-5


@pytest.mark.parametrize("batch,m,n", ROW_SHAPES[:5] + [(1, 8192, 3072)])
def test_gelu(cuda, batch, m, n):
    from cuda_autograd_fns import CudaGeluLayer
    from cuda_transformer.ops import gelu_activation, gelu_activation_bwd

    x = seeded((batch, m, n), 5, kind="rand") * 6 - 3  # covers the negative tail too
    dy = seeded((batch, m, n), 6, kind="rand")
    y = gelu_activation(x.to(cuda))
    np.testing.assert_allclose(f64(y), ew.gelu_forward(f64(x)), atol=1e-5, rtol=1e-5)
    dx = gelu_activation_bwd(x.to(cuda), dy.to(cuda))
    np.testing.assert_allclose(f64(dx), ew.gelu_backward(f64(x), f64(dy)), atol=1e-5, rtol=1e-5)
    xg = x.to(cuda).requires_grad_()
    CudaGeluLayer.apply(xg).backward(dy.to(cuda))
    assert torch.equal(xg.grad, dx)


def test_gelu_ragged_numel(cuda):
    from cuda_transformer.ops import gelu_activation

    for numel in (1, 3, 5, 1027):
        x = seeded((1, 1, numel), numel, kind="randn")
        np.testing.assert_allclose(f64(gelu_activation(x.to(cuda))), ew.gelu_forward(f64(x)),
                                   atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("batch,m,n", ROW_SHAPES[:5] + [(1, 8192, 3072)])
def test_gelu_tanh(cuda, batch, m, n):
    """The tanh-approximated GELU (config 4's GELU) against the float64 oracle, and the
    autograd class against the two ops."""
    from cuda_autograd_fns import CudaGeluTanhLayer
    from cuda_transformer.ops import gelu_tanh_activation, gelu_tanh_activation_bwd

    x = seeded((batch, m, n), 15, kind="rand") * 12 - 6
    dy = seeded((batch, m, n), 16, kind="rand")
    y = gelu_tanh_activation(x.to(cuda))
    np.testing.assert_allclose(f64(y), ew.gelu_tanh_forward(f64(x)), atol=1e-5, rtol=1e-5)
    dx = gelu_tanh_activation_bwd(x.to(cuda), dy.to(cuda))
    np.testing.assert_allclose(f64(dx), ew.gelu_tanh_backward(f64(x), f64(dy)), atol=1e-5,
                               rtol=1e-5)
    xg = x.to(cuda).requires_grad_()
    CudaGeluTanhLayer.apply(xg).backward(dy.to(cuda))
    assert torch.equal(xg.grad, dx)


def test_gelu_tanh_tails_and_ragged_numel(cuda):
    """Large |x| (where tanh saturates and x^3 is large), signed zeros, and sizes that are not
    a multiple of four (the scalar tail)."""
    from cuda_transformer.ops import gelu_tanh_activation, gelu_tanh_activation_bwd

    x = torch.tensor([-1e4, -100.0, -30.0, -9.0, -0.0, 0.0, 1e-30, 9.0, 30.0, 100.0, 1e4],
                     dtype=torch.float32)
    dy = torch.ones_like(x)
    y, dx = gelu_tanh_activation(x.to(cuda)), gelu_tanh_activation_bwd(x.to(cuda), dy.to(cuda))
    np.testing.assert_allclose(f64(y), ew.gelu_tanh_forward(f64(x)), atol=1e-6, rtol=1e-6)
    np.testing.assert_allclose(f64(dx), ew.gelu_tanh_backward(f64(x), f64(dy)), atol=1e-6,
                               rtol=1e-6)
    for numel in (1, 3, 5, 1027):
        x = seeded((1, 1, numel), numel, kind="randn") * 3
        dy = seeded((1, 1, numel), numel + 1, kind="randn")
        np.testing.assert_allclose(f64(gelu_tanh_activation(x.to(cuda))),
                                   ew.gelu_tanh_forward(f64(x)), atol=1e-6, rtol=1e-5)
        np.testing.assert_allclose(f64(gelu_tanh_activation_bwd(x.to(cuda), dy.to(cuda))),
                                   ew.gelu_tanh_backward(f64(x), f64(dy)), atol=1e-6, rtol=1e-5)


def test_gelu_tanh_through_c_abi(cuda):
    from cuda_transformer_amd import capi

    x = seeded((3, 1001), 21, kind="randn").to(cuda) * 2
    dy = seeded((3, 1001), 22, kind="randn").to(cuda)
    y, dx = torch.empty_like(x), torch.empty_like(x)
    stream = torch.cuda.current_stream().cuda_stream
    capi.call("cta_gelu_tanh_fwd", x.data_ptr(), y.data_ptr(), x.numel(), stream)
    capi.call("cta_gelu_tanh_bwd", x.data_ptr(), dy.data_ptr(), dx.data_ptr(), x.numel(), stream)
    torch.cuda.synchronize()
    np.testing.assert_allclose(f64(y), ew.gelu_tanh_forward(f64(x)), atol=1e-6, rtol=1e-5)
    np.testing.assert_allclose(f64(dx), ew.gelu_tanh_backward(f64(x), f64(dy)), atol=1e-6,
                               rtol=1e-5)


@pytest.mark.parametrize("batch,m,n", ROW_SHAPES + [(48, 1024, 1024)])
def test_softmax(cuda, batch, m, n):
    from cuda_autograd_fns import CudaSoftmaxLayer
    from cuda_transformer.ops import cuda_softmax, cuda_softmax_bwd

    scale = 2.0 if n == 1024 else 1.0  # config 4 logits ~ N(0, 4)
    x = seeded((batch, m, n), 7) * scale
    dp = seeded((batch, m, n), 8, kind="rand")
    p = cuda_softmax(x.to(cuda))
    p_ref = ew.softmax_forward(f64(x))
    np.testing.assert_allclose(f64(p), p_ref, atol=1e-5, rtol=1e-5)
    dx = cuda_softmax_bwd(p, dp.to(cuda))
    np.testing.assert_allclose(f64(dx), ew.softmax_backward(f64(p), f64(dp)), atol=1e-5,
                               rtol=1e-5)
    xg = x.to(cuda).requires_grad_()
    CudaSoftmaxLayer.apply(xg).backward(dp.to(cuda))
    assert torch.equal(xg.grad, dx)


@pytest.mark.parametrize("n", [70, 1024, 3000])  # scalar, float4 register path, long-row path
def test_softmax_large_magnitude_logits(cuda, n):
    """Rows whose maximum is huge: all -1e10 (a fully masked row), a maximum of 1e10, values
    near +-3e38, and rows that start with -inf (a mask before the first finite entry).  The
    exponent is (x - max) log2(e), so the maximum gets exactly e^0 at any magnitude; folding
    max log2(e) into one rounded offset would give inf or NaN on the first three."""
    from cuda_transformer.ops import cuda_softmax

    rng = np.random.default_rng(n)
    rows = np.zeros((6, n), np.float32)
    rows[0] = -1e10
    rows[1] = 1e10 - rng.integers(0, 4, n).astype(np.float32) * 2048.0  # 1e10 and its neighbours
    rows[2] = rng.choice(np.float32([3e38, 2.9e38, -3e38, 0.0]), n)
    rows[2, 0] = 3e38
    rows[3] = -3e38
    rows[3, n // 2] = -2.9e38
    rows[4] = rng.normal(0, 2, n).astype(np.float32)
    rows[4, : n // 3] = -np.inf
    rows[5] = rng.normal(0, 2, n).astype(np.float32) + 1e9
    x = torch.from_numpy(rows)[None]
    p = cuda_softmax(x.to(cuda))
    ref = ew.softmax_forward(rows.astype(np.float64))
    assert np.all(np.isfinite(ref))
    np.testing.assert_allclose(f64(p)[0], ref, atol=1e-6, rtol=1e-5)


def test_row_kernels_stride_past_the_grid_cap(cuda):
    """2^22 + 5 rows: more than the 2^20 four-row workgroups the softmax and LayerNorm-forward
    row kernels launch, so the last 5 rows come from a wave's second pass.  Rows at both ends
    and across the cap are checked against the oracle."""
    from cuda_transformer.ops import cuda_softmax, cuda_softmax_bwd, layernorm_fwd

    rows, n = (1 << 22) + 5, 4
    g = torch.Generator(device=cuda).manual_seed(7)
    x = torch.randn(1, rows, n, generator=g, device=cuda) * 2
    dp = torch.randn(1, rows, n, generator=g, device=cuda)
    gamma = torch.linspace(0.5, 1.5, n, device=cuda)
    beta = torch.linspace(-0.1, 0.1, n, device=cuda)
    p = cuda_softmax(x)
    dx = cuda_softmax_bwd(p, dp)
    y, mean, rstd = layernorm_fwd(x[0], gamma, beta, 1e-5)
    idx = torch.tensor([0, 1, (1 << 22) - 1, 1 << 22, rows - 3, rows - 1], device=cuda)
    xs, dps = f64(x[0, idx]), f64(dp[0, idx])
    ps = ew.softmax_forward(xs)
    np.testing.assert_allclose(f64(p[0, idx]), ps, atol=1e-6, rtol=1e-5)
    np.testing.assert_allclose(f64(dx[0, idx]), ew.softmax_backward(f64(p[0, idx]), dps),
                               atol=1e-6, rtol=1e-5)
    y_r, mean_r, rstd_r = ew.layernorm_forward(xs, f64(gamma), f64(beta), 1e-5)
    np.testing.assert_allclose(f64(y[idx]), y_r, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(f64(mean[idx]), mean_r.reshape(-1), atol=1e-6, rtol=1e-5)
    np.testing.assert_allclose(f64(rstd[idx]), rstd_r.reshape(-1), atol=1e-6, rtol=1e-4)
    # every row was written: each softmax row sums to one, every output is finite
    assert torch.allclose(p.sum(-1), torch.ones(1, rows, device=cuda), atol=1e-5)
    assert bool(torch.isfinite(y).all()) and bool(torch.isfinite(dx).all())


@pytest.mark.parametrize("rows,n", [(64, 32), (65, 32), (70, 120), (8192, 768), (33, 384),
                                    (5, 2048), (3, 3000), (7, 65)])
def test_layernorm(cuda, rows, n):
    from cuda_autograd_fns import CudaLayerNorm

    x = seeded((rows, n), 9) * 3 + 1
    gamma = 1 + 0.1 * seeded((n,), 10)
    beta = 0.1 * seeded((n,), 11)
    dy = seeded((rows, n), 12)
    xg, gg, bg = (t.to(cuda).requires_grad_() for t in (x, gamma, beta))
    y = CudaLayerNorm.apply(xg, gg, bg, 1e-5)
    y.backward(dy.to(cuda))
    y_ref, mean, rstd = ew.layernorm_forward(f64(x), f64(gamma), f64(beta), 1e-5)
    np.testing.assert_allclose(f64(y), y_ref, atol=1e-5, rtol=1e-5)
    dx_r, dg_r, db_r = ew.layernorm_backward(f64(x), f64(gamma), mean, rstd, f64(dy))
    np.testing.assert_allclose(f64(xg.grad), dx_r, atol=1e-4, rtol=1e-5)
    assert rel_err(f64(gg.grad), dg_r) <= 1e-5
    assert rel_err(f64(bg.grad), db_r) <= 1e-5


NAIVE_SHAPES = [(1, 64, 1, 32, False), (1, 64, 1, 32, True), (1, 65, 1, 32, True),
                (2, 128, 4, 64, False), (2, 128, 4, 64, True), (2, 257, 4, 64, True),
                (1, 512, 2, 128, True)]


@pytest.mark.parametrize("B,T,nh,hs,causal", NAIVE_SHAPES)
def test_causal_self_attention(cuda, B, T, nh, hs, causal):
    from cuda_autograd_fns import CudaCausalSelfAttention
    from cuda_transformer.ops import causal_self_attention_bwd, causal_self_attention_fwd

    C = nh * hs
    qkv = seeded((B, T, 3 * C), 13, kind="rand")
    dO = seeded((B, T, C), 14, kind="rand")
    out, probs = causal_self_attention_fwd(qkv.to(cuda), nh, causal)
    out_r, probs_r = ora.causal_self_attention_forward(f64(qkv), nh, causal)
    assert probs.shape == (B, nh, T, T)
    np.testing.assert_allclose(f64(out), out_r, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(f64(probs), probs_r, atol=1e-5, rtol=1e-5)

    def heads(t):
        return t.reshape(B, T, nh, hs).transpose(1, 2).reshape(B * nh, T, hs)

    q, k, v = (heads(t) for t in qkv.to(cuda).chunk(3, dim=-1))
    dq, dk, dv = causal_self_attention_bwd(q, k, v, probs.reshape(B * nh, T, T),
                                           heads(dO.to(cuda)))
    g_r = ora.causal_self_attention_backward(f64(q), f64(k), f64(v),
                                             probs_r.reshape(B * nh, T, T), f64(heads(dO)))
    for got, ref in zip((dq, dk, dv), g_r):
        np.testing.assert_allclose(f64(got), ref, atol=1e-4, rtol=1e-5)
    # autograd wrapper: grads of the packed qkv against the float64 oracle
    qg = qkv.to(cuda).requires_grad_()
    CudaCausalSelfAttention.apply(qg, nh, causal).backward(dO.to(cuda))
    sm = hs ** 0.5

    def unheads(a):
        return a.reshape(B, nh, T, hs).transpose(0, 2, 1, 3).reshape(B, T, C)

    ref_grad = np.concatenate([unheads(g_r[0]) / sm, unheads(g_r[1]) / sm, unheads(g_r[2])], -1)
    np.testing.assert_allclose(f64(qg.grad), ref_grad, atol=1e-4, rtol=1e-5)


@pytest.mark.parametrize("B,M,K,N", [(1, 100, 3000, 130), (2, 64, 4096, 96), (1, 768, 8192, 256)])
def test_linear_split_k(cuda, B, M, K, N):
    """Few output tiles and a long K: the GEMM splits K across workgroups (deterministic)."""
    from cuda_transformer.ops import cuda_fma
    from cuda_transformer_amd import capi

    assert capi.lib().cta_cuda_fma_workspace(B, M, K, N) > 0
    x = seeded((B, M, K), 31, kind="rand")
    w = seeded((K, N), 32) * 0.05
    b = seeded((N,), 33)
    out = cuda_fma(x.to(cuda), w.to(cuda), b.to(cuda))
    ref = lin.fma_forward(f64(x), f64(w), f64(b))
    assert rel_err(f64(out), ref) <= 1e-6
    out2 = cuda_fma(x.to(cuda), w.to(cuda), b.to(cuda))
    assert torch.equal(out, out2)
    # transposed operand view (the linear backward's x^T): (B, K, M) . (B, M, N)
    dyt = seeded((B, M, N), 34).to(cuda)
    out3 = cuda_fma(x.to(cuda).transpose(1, 2), dyt, torch.zeros(N, device=cuda))
    assert rel_err(f64(out3), np.swapaxes(f64(x), 1, 2) @ f64(dyt)) <= 1e-6


@pytest.mark.parametrize("M,K,N", [(96, 100, 68), (130, 36, 1152), (64, 1020, 388), (33, 4100, 64)])
def test_linear_ragged_k_vector_loads(cuda, M, K, N):
    """K not a multiple of the K-slice while both operands take 16-byte loads: the last slice's
    lanes past K must read zeros (forward x.W, dx = dy.W^T view, dW = x^T view . dy)."""
    from cuda_transformer.ops import cuda_fma

    x = seeded((1, M, K), 41).to(cuda)
    w = seeded((K, N), 42).to(cuda) * 0.1
    b = seeded((N,), 43).to(cuda)
    out = cuda_fma(x, w, b)
    assert rel_err(f64(out), f64(x) @ f64(w) + f64(b)) <= 1e-6
    wt = seeded((N, K), 44).to(cuda)                    # W stored (N, K): its W^T view is k-contiguous
    out = cuda_fma(x, wt.t().unsqueeze(0), torch.zeros(N, device=cuda))
    assert rel_err(f64(out), f64(x) @ f64(wt).T) <= 1e-6
    dy = seeded((1, M, N), 45).to(cuda)
    out = cuda_fma(x.transpose(1, 2), dy, torch.zeros(N, device=cuda))
    assert rel_err(f64(out), np.swapaxes(f64(x), 1, 2) @ f64(dy)) <= 1e-6


@pytest.mark.parametrize("B,M,K,N", [(64, 256, 384, 1152), (3, 130, 64, 200), (9, 16, 32, 8)])
def test_linear_batched_tiles_over_xcds(cuda, B, M, K, N):
    """Batched products spread the tiles of all batches over the XCDs as one list: every tile of
    every batch is computed once (batches with few tiles each, as in the GPT's layers)."""
    from cuda_transformer.ops import cuda_fma

    x = seeded((B, M, K), 51).to(cuda)
    w = seeded((K, N), 52).to(cuda) * 0.1
    b = seeded((N,), 53).to(cuda)
    out = cuda_fma(x, w, b)
    assert rel_err(f64(out), f64(x) @ f64(w) + f64(b)) <= 1e-6
    wb = seeded((B, K, N), 54).to(cuda)                 # per-batch weights
    out = cuda_fma(x, wb, b)
    assert rel_err(f64(out), f64(x) @ f64(wb) + f64(b)) <= 1e-6


# (B, M, K, N) with N a multiple of 192 (the 192-column tiles): short and long K, ragged M and
# K, one tile column, and N > 768
@pytest.mark.parametrize("B,M,K,N", [(1, 333, 200, 576), (2, 100, 700, 192), (1, 130, 37, 384),
                                     (1, 257, 1000, 768), (3, 70, 96, 960), (1, 200, 300, 1152)])
def test_linear_192_column_tiles(cuda, B, M, K, N):
    from cuda_transformer.ops import cuda_fma, cuda_fma_gelu

    x = seeded((B, M, K), 50).to(cuda)
    w = seeded((K, N), 51).to(cuda) * 0.1
    b = seeded((N,), 52).to(cuda)
    ref = lin.fma_forward(f64(x), f64(w), f64(b))
    assert rel_err(f64(cuda_fma(x, w, b)), ref) <= 1e-5
    pre, h = cuda_fma_gelu(x, w, b)
    assert torch.equal(pre, cuda_fma(x, w, b))
    np.testing.assert_allclose(f64(h), ew.gelu_forward(f64(pre)), atol=1e-5, rtol=1e-5)
    # transposed operands (the linear backward's dx and dW views)
    dy = seeded((B, M, N), 53).to(cuda)
    dx = cuda_fma(dy, w.unsqueeze(0).transpose(1, 2), torch.zeros(K, device=cuda))
    assert rel_err(f64(dx), f64(dy) @ f64(w).T) <= 1e-5


def test_linear_operand_strides_past_buffer_offsets(cuda):
    """Operand views whose strides put a tile's rows more than 2 GiB apart cannot be addressed
    with 32-bit buffer offsets; they take the scalar load path and stay exact."""
    from cuda_transformer.ops import cuda_fma

    M, K, N = 5, 64, 48
    big = torch.zeros(M, 2_200_000, device=cuda)
    big[:, :K] = seeded((M, K), 46).to(cuda)
    x = big[:, :K].unsqueeze(0)                         # row stride 2.2e6 floats
    w = seeded((K, N), 47).to(cuda)
    b = seeded((N,), 48).to(cuda)
    out = cuda_fma(x, w, b)
    assert rel_err(f64(out), f64(x) @ f64(w) + f64(b)) <= 1e-6
    wbig = torch.zeros(K, 9_000_000, device=cuda)       # W (K, N) view with k stride 9e6 floats
    wbig[:, :N] = w
    out2 = cuda_fma(x, wbig[:, :N], b)
    assert torch.equal(out2, out)
    del big, wbig


def test_db_strided_views(cuda):
    from cuda_transformer.ops import db_calculation

    base = seeded((3, 50, 70), 35).to(cuda)
    for dy in (base, base[:, 5:45, :], base.transpose(1, 2), base[:, :, 3:67]):
        got = db_calculation(dy)
        np.testing.assert_allclose(f64(got), f64(dy).sum(axis=(0, 1)), rtol=1e-5, atol=1e-4)
    big = seeded((2, 4100, 1030), 36).to(cuda)
    np.testing.assert_allclose(f64(db_calculation(big)), f64(big).sum(axis=(0, 1)), rtol=1e-5,
                               atol=1e-3)
    assert torch.equal(db_calculation(big), db_calculation(big))


# (rows, k, n): split-K with the SplitTile (GPT qkv / fc2 weight gradients, config 4), one
# unsplit 128x128-tile GEMM (256 tiles), unsplit narrow tiles with ragged rows, the unsplit
# 192-column tiles (64x192 with K-slices of 16 and 32, 128x192), and n % 4 != 0 (dy not
# vector-loadable: GEMM then the column-sum kernels).
WB_SHAPES = [(16384, 384, 1152), (16384, 1536, 384), (8192, 768, 3072), (2048, 2048, 2048),
             (333, 64, 100), (1000, 20, 36), (300, 64, 192), (800, 128, 384), (1000, 256, 1152),
             (100, 48, 65), (5, 7, 12)]


@pytest.mark.parametrize("rows,k,n", WB_SHAPES)
def test_linear_weight_bias_grad(cuda, rows, k, n):
    # dW bitwise equal to the cuda_fma route (same kernel schedule, same K split); db checked
    # against the float64 oracle, and reproducible call to call.
    from cuda_transformer.ops import cuda_fma
    from cuda_transformer_amd.ops import linear_weight_bias_grad

    x = seeded((rows, k), 40).to(cuda)
    dy = seeded((rows, n), 41).to(cuda)
    dw, db = linear_weight_bias_grad(x, dy)
    ref_dw = cuda_fma(x.unsqueeze(0).transpose(1, 2), dy.unsqueeze(0), torch.zeros(n, device=cuda))[0]
    assert torch.equal(dw, ref_dw)
    _, dw_r, db_r = lin.linear_backward(f64(x)[None], np.zeros((k, n)), f64(dy)[None])
    assert rel_err(f64(dw), dw_r) <= 1e-5
    scale = np.abs(f64(dy)).sum(axis=0)
    assert np.all(np.abs(f64(db) - db_r) <= 1e-6 * scale + 1e-6)
    dw2, db2 = linear_weight_bias_grad(x, dy)
    assert torch.equal(dw, dw2) and torch.equal(db, db2)


def test_linear_weight_bias_grad_views_and_edges(cuda):
    from cuda_transformer.ops import cuda_fma
    from cuda_transformer_amd.ops import linear_weight_bias_grad

    # x as a transposed view (k-contiguous A), dy rows strided past n, a 3-D batch folded into
    # the rows, and a misaligned dy base (no vector loads: unfused path)
    xt = seeded((96, 3000), 42).to(cuda)
    dyb = seeded((3000, 200), 43).to(cuda)
    cases = [(xt.t(), dyb[:, :128]), (seeded((3, 70, 40), 44).to(cuda), seeded((3, 70, 52), 45).to(cuda)),
             (seeded((257, 33), 46).to(cuda), dyb[:257, 1:129])]
    for x, dy in cases:
        dw, db = linear_weight_bias_grad(x, dy)
        x2, d2 = f64(x).reshape(-1, x.shape[-1]), f64(dy).reshape(-1, dy.shape[-1])
        assert rel_err(f64(dw), x2.T @ d2) <= 1e-5
        np.testing.assert_allclose(f64(db), d2.sum(axis=0), rtol=1e-5, atol=1e-4)
        ref = cuda_fma(x.reshape(1, -1, x.shape[-1]).transpose(1, 2), dy.reshape(1, -1, dy.shape[-1]),
                       torch.zeros(dy.shape[-1], device=cuda))[0]
        assert torch.equal(dw, ref)
    # zero rows: both gradients are zero; zero k: db alone
    dw, db = linear_weight_bias_grad(torch.empty(0, 5, device=cuda), torch.empty(0, 8, device=cuda))
    assert torch.equal(dw.cpu(), torch.zeros(5, 8)) and torch.equal(db.cpu(), torch.zeros(8))
    dy = seeded((300, 8), 47).to(cuda)
    dw, db = linear_weight_bias_grad(torch.empty(300, 0, device=cuda), dy)
    assert dw.shape == (0, 8)
    np.testing.assert_allclose(f64(db), f64(dy).sum(axis=0), rtol=1e-5, atol=1e-5)
    with pytest.raises(RuntimeError, match="every dim but the last"):
        linear_weight_bias_grad(torch.empty(4, 5, device=cuda), torch.empty(3, 8, device=cuda))


# ------------------------------------------------------------ fused linear + GELU (GPT MLP)
# (batch, rows, d, hidden); the last shape has 1 output tile and K = 4096, so it runs split-K.
FUSED_SHAPES = [(1, 32, 64, 96), (2, 33, 17, 65), (3, 70, 129, 257), (2, 256, 384, 1536),
                (1, 64, 4096, 96)]


def _gelu_forms(form):
    """(fused fwd, fused grad, plain fwd, plain bwd, oracle fwd, oracle bwd) of one GELU form."""
    from cuda_transformer import ops

    if form == "erf":
        return (ops.cuda_fma_gelu, ops.cuda_fma_gelu_grad, ops.gelu_activation,
                ops.gelu_activation_bwd, ew.gelu_forward, ew.gelu_backward)
    return (ops.cuda_fma_gelu_tanh, ops.cuda_fma_gelu_tanh_grad, ops.gelu_tanh_activation,
            ops.gelu_tanh_activation_bwd, ew.gelu_tanh_forward, ew.gelu_tanh_backward)


def _gelu_deriv_form(form):
    from cuda_transformer import ops

    return ops.cuda_fma_gelu_deriv if form == "erf" else ops.cuda_fma_gelu_tanh_deriv


@pytest.mark.parametrize("form", ["erf", "tanh"])
@pytest.mark.parametrize("B,T,d,hid", FUSED_SHAPES)
def test_fused_linear_gelu(cuda, B, T, d, hid, form):
    """cuda_fma_gelu[_tanh] and cuda_fma_gelu[_tanh]_grad: the same bits as the unfused ops, and
    the oracle."""
    from cuda_transformer.ops import cuda_fma

    cuda_fma_gelu, cuda_fma_gelu_grad, gelu_activation, gelu_activation_bwd, o_fwd, o_bwd = (
        _gelu_forms(form))

    x = seeded((B, T, d), 50, kind="rand")
    w1 = seeded((d, hid), 51) * 0.2
    b1 = seeded((hid,), 52) * 0.2
    w2 = seeded((hid, d), 53) * 0.2
    dz = seeded((B, T, d), 54)
    xc, w1c, b1c, w2c, dzc = (t.to(cuda) for t in (x, w1, b1, w2, dz))
    pre, h = cuda_fma_gelu(xc, w1c, b1c)
    assert torch.equal(pre, cuda_fma(xc, w1c, b1c))
    assert torch.equal(h, gelu_activation(pre))
    # FP32 sums of up to K = 4096 terms: relative error in norm, and a looser elementwise bound
    pre_r = f64(x) @ f64(w1) + f64(b1)
    h_r = o_fwd(pre_r)
    w2t = w2c.unsqueeze(0).transpose(1, 2)
    dpre = cuda_fma_gelu_grad(dzc, w2t, pre)
    unfused = gelu_activation_bwd(pre, cuda_fma(dzc, w2t, torch.zeros(hid, device=cuda)))
    assert torch.equal(dpre, unfused)
    dpre_r = o_bwd(f64(pre), f64(dz) @ f64(w2).T)
    for got, ref in ((pre, pre_r), (h, h_r), (dpre, dpre_r)):
        assert rel_err(f64(got), ref) <= 1e-6
        np.testing.assert_allclose(f64(got), ref, atol=1e-4, rtol=1e-4)
    # The saved-derivative pair: GELU'(pre) from the forward epilogue, then a plain multiply in
    # the backward one; the same bits as the pair above.
    from cuda_transformer.ops import cuda_fma_mul

    deriv, h2 = _gelu_deriv_form(form)(xc, w1c, b1c)
    assert torch.equal(h2, h)
    assert torch.equal(deriv, gelu_activation_bwd(pre, torch.ones_like(pre)))
    assert torch.equal(cuda_fma_mul(dzc, w2t, deriv), dpre)
    np.testing.assert_allclose(f64(deriv), o_bwd(pre_r, np.ones_like(pre_r)), atol=1e-4,
                               rtol=1e-4)


def test_fused_linear_gelu_through_c_abi(cuda):
    """The C entry points: both outputs, the in-place gradient (dx aliasing pre), the error on
    pre == out."""
    from cuda_transformer.ops import cuda_fma_gelu, cuda_fma_gelu_grad
    from cuda_transformer_amd import capi

    B, T, d, hid = 2, 40, 48, 80
    x = seeded((B, T, d), 55).to(cuda)
    w1 = seeded((d, hid), 56).to(cuda) * 0.2
    b1 = seeded((hid,), 57).to(cuda)
    w2t = (seeded((hid, d), 58).to(cuda) * 0.2).t()      # (d, hid) view, strides (1, d)
    dz = seeded((B, T, d), 59).to(cuda)
    stream = torch.cuda.current_stream().cuda_stream
    pre = torch.empty(B, T, hid, device=cuda)
    out = torch.empty_like(pre)
    capi.call("cta_cuda_fma_gelu", x.data_ptr(), capi.strides(x.stride()), w1.data_ptr(),
              capi.strides((0,) + w1.stride()), b1.data_ptr(), 1, B, T, d, hid, 1,
              pre.data_ptr(), out.data_ptr(), None, stream)
    dx = pre.clone()
    capi.call("cta_cuda_fma_gelu_grad", dz.data_ptr(), capi.strides(dz.stride()), w2t.data_ptr(),
              capi.strides((0,) + w2t.stride()), dx.data_ptr(), B, T, d, hid, 1, dx.data_ptr(),
              None, stream)
    torch.cuda.synchronize()
    pre_t, out_t = cuda_fma_gelu(x, w1, b1)
    assert torch.equal(pre, pre_t) and torch.equal(out, out_t)
    assert torch.equal(dx, cuda_fma_gelu_grad(dz, w2t, pre_t))
    with pytest.raises(capi.CtaError, match="distinct"):
        capi.call("cta_cuda_fma_gelu", x.data_ptr(), capi.strides(x.stride()), w1.data_ptr(),
                  capi.strides((0,) + w1.stride()), b1.data_ptr(), 1, B, T, d, hid, 1,
                  pre.data_ptr(), pre.data_ptr(), None, stream)


def test_fused_linear_gelu_tanh_through_c_abi(cuda):
    from cuda_transformer.ops import cuda_fma_gelu_tanh, cuda_fma_gelu_tanh_grad
    from cuda_transformer_amd import capi

    B, T, d, hid = 2, 40, 48, 80
    x = seeded((B, T, d), 75).to(cuda)
    w1 = seeded((d, hid), 76).to(cuda) * 0.2
    b1 = seeded((hid,), 77).to(cuda)
    w2t = (seeded((hid, d), 78).to(cuda) * 0.2).t()
    dz = seeded((B, T, d), 79).to(cuda)
    stream = torch.cuda.current_stream().cuda_stream
    pre = torch.empty(B, T, hid, device=cuda)
    out = torch.empty_like(pre)
    capi.call("cta_cuda_fma_gelu_tanh", x.data_ptr(), capi.strides(x.stride()), w1.data_ptr(),
              capi.strides((0,) + w1.stride()), b1.data_ptr(), 1, B, T, d, hid, 1,
              pre.data_ptr(), out.data_ptr(), None, stream)
    dx = pre.clone()
    capi.call("cta_cuda_fma_gelu_tanh_grad", dz.data_ptr(), capi.strides(dz.stride()),
              w2t.data_ptr(), capi.strides((0,) + w2t.stride()), dx.data_ptr(), B, T, d, hid, 1,
              dx.data_ptr(), None, stream)
    torch.cuda.synchronize()
    pre_t, out_t = cuda_fma_gelu_tanh(x, w1, b1)
    assert torch.equal(pre, pre_t) and torch.equal(out, out_t)
    assert torch.equal(dx, cuda_fma_gelu_tanh_grad(dz, w2t, pre_t))


@pytest.mark.parametrize("form", ["erf", "tanh"])
def test_fused_linear_gelu_deriv_through_c_abi(cuda, form):
    """cta_cuda_fma_gelu[_tanh]_deriv and cta_cuda_fma_mul with dx aliasing the derivative: the
    same bits as the pre-activation pair, and the error on deriv == out."""
    from cuda_transformer import ops
    from cuda_transformer_amd import capi

    fwd, grad = ((ops.cuda_fma_gelu, ops.cuda_fma_gelu_grad) if form == "erf"
                 else (ops.cuda_fma_gelu_tanh, ops.cuda_fma_gelu_tanh_grad))
    entry = "cta_cuda_fma_gelu_deriv" if form == "erf" else "cta_cuda_fma_gelu_tanh_deriv"
    B, T, d, hid = 2, 40, 48, 80
    x = seeded((B, T, d), 85).to(cuda)
    w1 = seeded((d, hid), 86).to(cuda) * 0.2
    b1 = seeded((hid,), 87).to(cuda)
    w2t = (seeded((hid, d), 88).to(cuda) * 0.2).t()
    dz = seeded((B, T, d), 89).to(cuda)
    stream = torch.cuda.current_stream().cuda_stream
    deriv = torch.empty(B, T, hid, device=cuda)
    out = torch.empty_like(deriv)
    capi.call(entry, x.data_ptr(), capi.strides(x.stride()), w1.data_ptr(),
              capi.strides((0,) + w1.stride()), b1.data_ptr(), 1, B, T, d, hid, 1,
              deriv.data_ptr(), out.data_ptr(), None, stream)
    dx = deriv.clone()
    capi.call("cta_cuda_fma_mul", dz.data_ptr(), capi.strides(dz.stride()), w2t.data_ptr(),
              capi.strides((0,) + w2t.stride()), dx.data_ptr(), B, T, d, hid, 1, dx.data_ptr(),
              None, stream)
    torch.cuda.synchronize()
    pre_t, out_t = fwd(x, w1, b1)
    assert torch.equal(out, out_t)
    assert torch.equal(dx, grad(dz, w2t, pre_t))
    with pytest.raises(RuntimeError, match="d must have shape"):
        ops.cuda_fma_mul(dz, w2t, deriv[:, :5])
    with pytest.raises(capi.CtaError, match="distinct"):
        capi.call(entry, x.data_ptr(), capi.strides(x.stride()), w1.data_ptr(),
                  capi.strides((0,) + w1.stride()), b1.data_ptr(), 1, B, T, d, hid, 1,
                  out.data_ptr(), out.data_ptr(), None, stream)


@pytest.mark.parametrize("tanh", [False, True])
@pytest.mark.parametrize("B,T,d", [(2, 33, 48), (4, 256, 384)])
def test_cuda_mlp_matches_composition(cuda, B, T, d, tanh):
    """CudaMLP: output and all five gradients bitwise equal to CudaLinearLayer -> CudaGeluLayer
    (CudaGeluTanhLayer with tanh=True) -> CudaLinearLayer, and within FP32 rounding of the
    oracle."""
    from cuda_autograd_fns import CudaGeluLayer, CudaGeluTanhLayer, CudaLinearLayer, CudaMLP

    hid = 4 * d
    params = [seeded(s, 60 + i) * 0.1 for i, s in enumerate([(d, hid), (hid,), (hid, d), (d,)])]
    x = seeded((B, T, d), 66)
    dz = seeded((B, T, d), 67)

    def run(fused):
        xg = x.to(cuda).requires_grad_()
        ps = [p.to(cuda).requires_grad_() for p in params]
        if fused:
            out = CudaMLP.apply(xg, *ps, tanh) if tanh else CudaMLP.apply(xg, *ps)
        else:
            act = CudaGeluTanhLayer if tanh else CudaGeluLayer
            h = act.apply(CudaLinearLayer.apply(xg, ps[0], ps[1]))
            out = CudaLinearLayer.apply(h, ps[2], ps[3])
        out.backward(dz.to(cuda))
        return [out.detach(), xg.grad] + [p.grad for p in ps]

    fused, plain = run(True), run(False)
    for a, b in zip(fused, plain):
        assert torch.equal(a, b)
    if tanh:
        return  # the tanh composition's parts are each checked against the oracle above
    p64 = [f64(p) for p in params]
    pre, h, out = lin.mlp_forward(f64(x), *p64)
    grads = lin.mlp_backward(f64(x), p64[0], p64[2], pre, h, f64(dz))
    assert rel_err(f64(fused[0]), out) <= 1e-5
    for g, r in zip(fused[1:], grads):
        assert rel_err(f64(g), r) <= 1e-5


def test_reductions_over_zero_rows_are_zero(cuda):
    # db and dgamma/dbeta over zero rows are sums over nothing: zeros, written by a fill
    # kernel into outputs that start out holding garbage.
    from cuda_transformer_amd import capi

    lib = capi.lib()
    st = torch.cuda.current_stream().cuda_stream
    db = torch.full((7,), float("nan"), device=cuda)
    s3 = capi.strides((0, 7, 1))
    assert lib.cta_db_calculation(None, s3, 1, 0, 7, db.data_ptr(), None, st) == 0
    dg = torch.full((5,), float("nan"), device=cuda)
    dbt = torch.full((5,), 3.0, device=cuda)
    assert lib.cta_layernorm_bwd(None, None, None, None, None, 0, 5, None, dg.data_ptr(),
                                 dbt.data_ptr(), None, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(db.cpu(), torch.zeros(7))
    assert torch.equal(dg.cpu(), torch.zeros(5)) and torch.equal(dbt.cpu(), torch.zeros(5))


@pytest.mark.parametrize("rows,n", [(64, 384), (33, 768), (70, 120), (9, 70), (5, 3000), (4, 2048)])
def test_add_layernorm_matches_add_then_layernorm(cuda, rows, n):
    # the fused residual add + LayerNorm against x + f then layernorm_fwd, and its backward
    # against layernorm_bwd then + dres: bit for bit (register path with float4 and scalar
    # rows, and the long-row path), and the float64 oracle
    from cuda_transformer_amd.ops import (add_layernorm_bwd, add_layernorm_fwd, layernorm_bwd,
                                          layernorm_fwd)

    x = seeded((rows, n), 60).to(cuda)
    f = seeded((rows, n), 61).to(cuda)
    gamma = (1.0 + 0.1 * seeded((n,), 62)).to(cuda)
    beta = (0.1 * seeded((n,), 63)).to(cuda)
    dy = seeded((rows, n), 64).to(cuda)
    dres = seeded((rows, n), 65).to(cuda)
    xs, y, mean, rstd = add_layernorm_fwd(x, f, gamma, beta, 1e-5)
    y2, mean2, rstd2 = layernorm_fwd(x + f, gamma, beta, 1e-5)
    assert torch.equal(xs, x + f)
    assert torch.equal(y, y2) and torch.equal(mean, mean2) and torch.equal(rstd, rstd2)
    y_r, mean_r, rstd_r = ew.layernorm_forward(f64(x) + f64(f), f64(gamma), f64(beta), 1e-5)
    np.testing.assert_allclose(f64(y), y_r, atol=2e-5, rtol=1e-5)
    dx_r, dg_r, db_r = ew.layernorm_backward(f64(x) + f64(f), f64(gamma), mean_r, rstd_r, f64(dy))
    dx, dg, db = add_layernorm_bwd(xs, gamma, mean, rstd, dy, dres)
    dx2, dg2, db2 = layernorm_bwd(xs, gamma, mean, rstd, dy)
    assert torch.equal(dx, dx2 + dres)
    assert torch.equal(dg, dg2) and torch.equal(db, db2)
    np.testing.assert_allclose(f64(dx), dx_r + f64(dres), atol=1e-4, rtol=1e-5)
    np.testing.assert_allclose(f64(dg), dg_r, atol=1e-4, rtol=1e-5)


def test_add_layernorm_autograd(cuda):
    # CudaAddLayerNorm's gradients against x + f -> CudaLayerNorm with autograd summing the two
    # paths, bit for bit; an unused xsum output leaves the plain LayerNorm backward
    from cuda_autograd_fns import CudaAddLayerNorm, CudaLayerNorm

    x0 = seeded((4, 16, 384), 66).to(cuda)
    f0 = seeded((4, 16, 384), 67).to(cuda)
    g0 = (1.0 + 0.1 * seeded((384,), 68)).to(cuda)
    b0 = (0.1 * seeded((384,), 69)).to(cuda)
    gy = seeded((4, 16, 384), 70).to(cuda)
    gs = seeded((4, 16, 384), 71).to(cuda)
    grads = []
    for fused in (True, False):
        x, f, g, b = (t.clone().requires_grad_() for t in (x0, f0, g0, b0))
        if fused:
            xs, y = CudaAddLayerNorm.apply(x, f, g, b, 1e-5)
        else:
            xs = x + f
            y = CudaLayerNorm.apply(xs, g, b, 1e-5)
        torch.autograd.backward([xs, y], [gs, gy])
        grads.append([t.grad for t in (x, f, g, b)])
    for a, r in zip(*grads):
        assert torch.equal(a, r)
    x, f, g, b = (t.clone().requires_grad_() for t in (x0, f0, g0, b0))
    _, y = CudaAddLayerNorm.apply(x, f, g, b, 1e-5)
    y.backward(gy)
    xr, fr, gr, br = (t.clone().requires_grad_() for t in (x0, f0, g0, b0))
    CudaLayerNorm.apply(xr + fr, gr, br, 1e-5).backward(gy)
    assert torch.equal(x.grad, xr.grad) and torch.equal(f.grad, fr.grad)
    assert torch.equal(g.grad, gr.grad) and torch.equal(b.grad, br.grad)


def test_device_copy(cuda):
    from cuda_transformer_amd import capi

    src = seeded((3 * 1024 * 1024 + 4,), 90).to(cuda)
    dst = torch.full_like(src, float("nan"))
    capi.call("cta_device_copy", src.data_ptr(), dst.data_ptr(), src.numel(),
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
    with pytest.raises(capi.CtaError, match="n % 4 == 0"):
        capi.call("cta_device_copy", src.data_ptr(), dst.data_ptr(), 6, 0)


def test_cuda_fma_rows_beyond_32bit_offsets(cuda):
    """Output rows of 2^24 + 4 floats: a wave's block of rows then spans more than 2^31 bytes,
    which the epilogue's 32-bit buffer offsets cannot address, so it stores through 64-bit
    addresses.  x (1, 2, 4) . W (4, N) + b against the float64 product; the fused GELU epilogue
    on the same product gives the same pre-activation bits and GELU(pre)."""
    from cuda_transformer.ops import cuda_fma
    from cuda_transformer_amd.ops import cuda_fma_gelu

    N = (1 << 24) + 4
    print(f"cuda_fma M2 K4 N{N}", flush=True)
    x = seeded((1, 2, 4), 101).to(cuda)
    w = seeded((4, N), 102).to(cuda)
    b = seeded((N,), 103).to(cuda)
    out = cuda_fma(x, w, b)
    pre, act = cuda_fma_gelu(x, w, b)
    torch.cuda.synchronize()
    ref = f64(x)[0] @ f64(w) + f64(b)
    np.testing.assert_allclose(f64(out)[0], ref, rtol=1e-5, atol=1e-5)
    assert torch.equal(pre, out)
    np.testing.assert_allclose(f64(act)[0], ew.gelu_forward(ref), rtol=1e-5, atol=1e-5)
    del w, out, pre, act
