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


@pytest.mark.parametrize("flag", ["fused_mlp", "fused_residual_ln"])
def test_gpt_fusions_match_reference_composition(cuda, flag):
    """GPTConfig.fused_mlp (CudaMLP) against the reference's Linear -> GELU -> Linear modules,
    and GPTConfig.fused_residual_ln (CudaAddLayerNorm) against separate residual adds and
    LayerNorms: the same loss and gradients, bit for bit (the embedding gradients, accumulated
    by torch's own embedding backward, to FP32 rounding)."""
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
