"""Benchmark config 5: the small GPT (6 layers, 6 heads, d_model 384, context 256, vocab 65,
batch 64) trained for 5 AdamW steps on the HIP kernels, against the same model in plain torch
on the CPU from identical weights and token ids.  Loss must match at every step."""
import pytest
import torch

from cuda_transformer_amd.gpt import GPT, GPTConfig, init_weights_, synthetic_batch
from oracle import gpt as ogpt

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fused_adamw", [False, True])  # the bench's step uses the fused AdamW
def test_gpt_training_steps_match_cpu_reference(cuda, fused_adamw):
    cfg = GPTConfig()
    model = GPT(cfg)
    ref = ogpt.GPT(cfg)
    init_weights_(model, seed=0)
    ref.load_state_dict(model.state_dict())
    model.to(cuda)
    opt = torch.optim.AdamW(model.parameters(), lr=6e-4, fused=fused_adamw)
    opt_ref = torch.optim.AdamW(ref.parameters(), lr=6e-4)
    torch.set_num_threads(min(16, torch.get_num_threads()))
    losses, losses_ref = [], []
    for step in range(5):
        idx, tgt = synthetic_batch(cfg, 64, seed=100 + step)
        opt.zero_grad(set_to_none=True)
        _, loss = model(idx.to(cuda), tgt.to(cuda))
        loss.backward()
        opt.step()
        opt_ref.zero_grad(set_to_none=True)
        _, loss_ref = ref(idx, tgt)
        loss_ref.backward()
        opt_ref.step()
        losses.append(loss.item())
        losses_ref.append(loss_ref.item())
        print(f"step {step}: loss {losses[-1]:.6f}  cpu reference {losses_ref[-1]:.6f}", flush=True)
    for a, b in zip(losses, losses_ref):
        assert abs(a - b) <= 1e-4 * abs(b), (losses, losses_ref)
    assert losses[-1] < losses[0]  # it trains
    # parameters stay close after 5 updates
    for (name, p), q in zip(model.named_parameters(), ref.parameters()):
        torch.testing.assert_close(p.detach().cpu(), q.detach(), rtol=1e-3, atol=1e-4, msg=name)


@pytest.mark.parametrize("flag", ["fused_mlp", "fused_residual_ln", "cuda_embedding"])
def test_gpt_fusions_match_reference_composition(cuda, flag):
    """GPTConfig.fused_mlp (CudaMLP) against the reference's Linear -> GELU -> Linear modules,
    GPTConfig.fused_residual_ln (CudaAddLayerNorm) against separate residual adds and
    LayerNorms, and GPTConfig.cuda_embedding (CudaEmbedding) against nn.Embedding: the same
    loss and gradients, bit for bit (the embedding gradients, summed in different orders, to
    FP32 rounding)."""
    cfg = GPTConfig(n_layers=2)
    idx, tgt = synthetic_batch(cfg, 8, seed=7)
    runs = []
    for fused in (True, False):
        model = GPT(GPTConfig(n_layers=2, **{flag: fused}))
        init_weights_(model, seed=3)
        model.to(cuda)
        _, loss = model(idx.to(cuda), tgt.to(cuda))
        loss.backward()
        runs.append((loss.detach(), {n: p.grad for n, p in model.named_parameters()}))
    (loss_f, g_f), (loss_u, g_u) = runs
    assert torch.equal(loss_f, loss_u)
    for name, g in g_f.items():
        if "embedding" in name or "positional" in name:
            torch.testing.assert_close(g, g_u[name], rtol=1e-6, atol=1e-7, msg=name)
        else:
            assert torch.equal(g, g_u[name]), name


@pytest.mark.parametrize("limit", [None, 0])  # the one-hot GEMM, then torch's backward
def test_cuda_embedding(cuda, limit, monkeypatch):
    """CudaEmbedding: the forward equals nn.Embedding's lookups; the table gradients match a
    float64 sum (and, through the fallback, torch's embedding backward bit for bit); re-runs are
    bitwise equal; position rows past T get zero gradient."""
    import torch.nn.functional as F

    from cuda_transformer_amd.autograd_fns import CudaEmbedding

    if limit is not None:
        monkeypatch.setattr(CudaEmbedding, "ONEHOT_LIMIT", limit)
    V, P, C, B, T = 65, 40, 48, 5, 33
    g = torch.Generator().manual_seed(11)
    tokens = torch.randint(0, V, (B, T), generator=g).to(cuda)
    tokens[0, :7] = 3                                   # a repeated id, and ids that never occur
    wte = torch.randn(V, C, generator=g).to(cuda).requires_grad_()
    wpe = torch.randn(P, C, generator=g).to(cuda).requires_grad_()
    dy = torch.randn(B, T, C, generator=g).to(cuda)
    out = CudaEmbedding.apply(tokens, wte, wpe)
    assert torch.equal(out, F.embedding(tokens, wte) + F.embedding(torch.arange(T, device=cuda), wpe))
    grads = []
    for _ in range(2):
        wte.grad = wpe.grad = None
        CudaEmbedding.apply(tokens, wte, wpe).backward(dy)
        grads.append((wte.grad.clone(), wpe.grad.clone()))
    assert all(torch.equal(a, b) for a, b in zip(grads[0], grads[1]))
    dwte, dwpe = grads[0]
    ids, dy64 = tokens.reshape(-1).cpu(), dy.reshape(-1, C).double().cpu()
    ref_te = torch.zeros(V, C, dtype=torch.float64).index_add_(0, ids, dy64)
    torch.testing.assert_close(dwte.double().cpu(), ref_te, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(dwpe[:T].double().cpu(), dy.double().sum(0).cpu(), rtol=1e-6,
                               atol=1e-6)
    assert torch.count_nonzero(dwpe[T:]) == 0
    if limit == 0:
        torch_te = torch.ops.aten.embedding_dense_backward(dy.reshape(-1, C), tokens.reshape(-1),
                                                           V, -1, False)
        assert torch.equal(dwte, torch_te)
    wte.grad = None
    CudaEmbedding.apply(tokens.to(torch.int32), wte, wpe).backward(dy)  # int32 ids
    assert torch.equal(wte.grad, dwte)
