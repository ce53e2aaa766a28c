"""FlashAttention-2 with 16-bit (bfloat16 and float16) Q, K, V on the GPU vs the CPU oracle
(float64).

The oracle is evaluated on the 16-bit-rounded inputs, so input rounding is not counted as kernel
error.  The kernel accumulates in FP32 and rounds twice: the probabilities to 16 bits as the
P.V operand, and O on output, each a relative error of at most 2^-9 for bfloat16 (2^-12 for
float16).  Hence per element
    |O - O_ref| <= 2^-9 |O_ref| + 2^-9 max_j |v_j| (+ FP32 accumulation),
bounded here by 2^-8 (|O_ref| + max|V|) for both types; L comes from FP32 scores of exact
16-bit products and keeps an FP32-level bound of 1e-4.  Shapes follow the FP32 suite (ragged T,
causal and full, hs 32, 64 and 128, benchmark config 1).
"""
import numpy as np
import pytest
import torch

from conftest import f64, seeded
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16]

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
    (2, 4, 128, 32, False),  # hs = 32 (the reference suite's (2, 4, 128, 32) shape)
    (2, 2, 129, 32, True),
    (1, 3, 300, 32, True),
]


def _half_inputs(B, nh, T, hs, seed, dtype=torch.bfloat16):
    return [seeded((B, nh, T, hs), seed + i).to(dtype) for i in range(3)]


def _check(O, L, q, k, v, causal):
    O_ref, L_ref = ora.reference_attention(f64(q), f64(k), f64(v), causal)
    assert O.dtype == q.dtype and L.dtype == torch.float32
    bound = 2.0 ** -8 * (np.abs(O_ref) + np.abs(f64(v)).max())
    err = np.abs(f64(O) - O_ref)
    assert (err <= bound).all(), f"O error {err.max():.3e} exceeds the bf16 bound"
    assert np.abs(f64(L) - L_ref).max() <= 1e-4
    return err.max()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,nh,T,hs,causal", SHAPES)
def test_fa2_half_forward_matches_oracle(cuda, B, nh, T, hs, causal, dtype):
    from cuda_transformer.ops import flash_attention_fwd

    q, k, v = _half_inputs(B, nh, T, hs, seed=3000 + T + hs, dtype=dtype)
    O, L = flash_attention_fwd(q.to(cuda), k.to(cuda), v.to(cuda), causal)
    torch.cuda.synchronize()
    _check(O.cpu(), L.cpu(), q, k, v, causal)


@pytest.mark.parametrize("dtype", DTYPES)
def test_fa2_half_forward_error_like_torch(cuda, dtype):
    """The kernel's error against the float64 oracle is no larger than that of torch's own
    16-bit attention (CPU SDPA on the same inputs)."""
    import torch.nn.functional as F

    from cuda_transformer.ops import flash_attention_fwd

    q, k, v = _half_inputs(1, 4, 256, 64, seed=77, dtype=dtype)
    O, _ = flash_attention_fwd(q.to(cuda), k.to(cuda), v.to(cuda), True)
    O_ref, _ = ora.reference_attention(f64(q), f64(k), f64(v), True)
    ours = np.abs(f64(O) - O_ref).mean()
    torch_bf16 = np.abs(f64(F.scaled_dot_product_attention(q, k, v, is_causal=True)) - O_ref).mean()
    assert ours <= 1.5 * torch_bf16 + 1e-4, (ours, torch_bf16)


def test_fa2_half_strided_views(cuda):
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


def test_fa2_half_deterministic(cuda):
    from cuda_transformer.ops import flash_attention_fwd

    q, k, v = (t.to(cuda) for t in _half_inputs(2, 4, 300, 128, seed=11))
    O1, L1 = flash_attention_fwd(q, k, v, True)
    O2, L2 = flash_attention_fwd(q, k, v, True)
    assert torch.equal(O1, O2) and torch.equal(L1, L2)


def test_fa2_half_errors(cuda):
    from cuda_transformer.ops import flash_attention_fwd

    q = torch.randn(1, 2, 16, 48, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="Only hs=32, hs=64, and hs=128 are supported"):
        flash_attention_fwd(q, q, q, False)
    q = torch.randn(1, 2, 16, 64, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="same dtype"):
        flash_attention_fwd(q, q.float(), q, False)
    with pytest.raises(RuntimeError, match="same dtype"):
        flash_attention_fwd(q, q.half(), q, False)


# ---------------------------------------------------------------- backward
# The oracle backward runs in float64 on the 16-bit-rounded q, k, v, dO with the exact O and L.
# The kernel rounds P and dS to 16 bits as MFMA operands (2^-9 relative each for bfloat16),
# forms delta from its 16-bit O, and rounds the gradients on output.  dV carries only the P rounding and
# its own output rounding; dQ and dK also the dS rounding, where dP - delta can cancel.  Bounds
# on the relative L2 error: 1.5e-2 for dV, 3e-2 for dQ and dK.
BWD_SHAPES = [
    (1, 4, 256, 64, True),   # benchmark config 1
    (1, 4, 256, 64, False),  # benchmark config 1
    (1, 1, 65, 64, True),
    (2, 4, 257, 64, True),
    (1, 2, 200, 128, False),
    (1, 2, 512, 128, True),
    (1, 3, 1, 64, True),
    (2, 2, 1000, 64, False),
    (2, 4, 128, 32, False),
    (2, 2, 129, 32, True),
    (1, 2, 600, 32, True),
]


def _bwd_check(grads, q, k, v, do, causal):
    from conftest import rel_err

    O_ref, L_ref = ora.reference_attention(f64(q), f64(k), f64(v), causal)
    refs = ora.fa2_backward(f64(q), f64(k), f64(v), O_ref, f64(do), L_ref, causal, br=64, bc=64)
    errs = []
    for got, ref, tol in zip(grads, refs, (3e-2, 3e-2, 1.5e-2)):
        assert got.dtype == q.dtype
        scale = 1e-6 * np.sqrt(ref.size)
        if np.linalg.norm(ref) <= scale:  # e.g. dQ for T = 1 is exactly zero
            assert np.linalg.norm(f64(got) - ref) <= 1e-3 * np.sqrt(ref.size)
            errs.append(0.0)
            continue
        e = rel_err(f64(got), ref)
        assert e <= tol, (e, tol)
        errs.append(e)
    return errs


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,nh,T,hs,causal", BWD_SHAPES)
def test_fa2_half_backward_matches_oracle(cuda, B, nh, T, hs, causal, dtype):
    from cuda_transformer.ops import flash_attention_bwd, flash_attention_fwd

    q, k, v = _half_inputs(B, nh, T, hs, seed=5000 + T + hs, dtype=dtype)
    do = seeded((B, nh, T, hs), 9000 + T, kind="rand").to(dtype)
    qg, kg, vg = q.to(cuda), k.to(cuda), v.to(cuda)
    O, L = flash_attention_fwd(qg, kg, vg, causal)
    grads = flash_attention_bwd(qg, kg, vg, O, do.to(cuda), L, causal)
    torch.cuda.synchronize()
    _bwd_check([g.cpu() for g in grads], q, k, v, do, causal)


@pytest.mark.parametrize("dtype", DTYPES)
def test_fa2_half_autograd_and_torch_error(cuda, dtype):
    """CudaFlashAttention with 16-bit leaves: gradients in the input dtype within the bounds
    above, and no more than twice the error of torch's own 16-bit SDPA backward (CPU) on the
    same inputs."""
    import torch.nn.functional as F

    from cuda_autograd_fns import CudaFlashAttention
    from conftest import rel_err

    B, nh, T, hs, causal = 1, 4, 256, 64, True
    q, k, v = _half_inputs(B, nh, T, hs, seed=41, dtype=dtype)
    do = seeded((B, nh, T, hs), 42, kind="rand").to(dtype)
    leaves = [t.to(cuda).requires_grad_() for t in (q, k, v)]
    o, _l = CudaFlashAttention.apply(*leaves, causal)
    o.backward(do.to(cuda))
    ours = _bwd_check([t.grad.cpu() for t in leaves], q, k, v, do, causal)

    tq, tk, tv = (t.clone().requires_grad_() for t in (q, k, v))
    F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal).backward(do)
    O_ref, L_ref = ora.reference_attention(f64(q), f64(k), f64(v), causal)
    refs = ora.fa2_backward(f64(q), f64(k), f64(v), O_ref, f64(do), L_ref, causal, br=64, bc=64)
    theirs = [rel_err(f64(t.grad), r) for t, r in zip((tq, tk, tv), refs)]
    for a, b in zip(ours, theirs):
        assert a <= 2.0 * b + 1e-3, (ours, theirs)


def test_fa2_half_backward_chunked_matches_full(cuda):
    """The head-chunked stored-dS schedule (a workspace of one head) gives the same bits as the
    full workspace."""
    import ctypes

    from cuda_transformer_amd import capi

    B, nh, T, hs = 2, 3, 300, 64
    q, k, v = (t.to(cuda) for t in _half_inputs(B, nh, T, hs, seed=61))
    from cuda_transformer.ops import flash_attention_fwd
    O, L = flash_attention_fwd(q, k, v, True)
    do = torch.rand(B, nh, T, hs, device=cuda).to(torch.bfloat16)
    lib = capi.lib()
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    s4, s3 = capi.strides(q.stride()), capi.strides(L.stride())
    outs = []
    for heads in (B * nh, 1):
        ws_bytes = lib.cta_flash_attention_bwd_bf16_workspace(1, 1, T, hs, 1) * heads
        ws = torch.empty(ws_bytes // 4 + 4, device=cuda)
        dq, dk, dv = (torch.empty_like(q) for _ in range(3))
        delta = torch.empty(B, nh, T, device=cuda)
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = lib.cta_flash_attention_bwd_bf16(P(q), s4, P(k), s4, P(v), s4, P(O), s4, P(do), s4,
                                              P(L), s3, B, nh, T, hs, 1, P(dq), P(dk), P(dv),
                                              P(delta), P(ws), ws_bytes, st)
        assert rc == 0, lib.cta_last_error()
        outs.append((dq, dk, dv))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


# ---------------------------------------------------------------- the two schedules
def _half_bwd_capi(q, k, v, O, do, L, causal, stored):
    """The 16-bit backward through the C ABI: the stored-dS schedule (a workspace for every
    head) or the recompute schedule (no workspace)."""
    import ctypes

    from cuda_transformer_amd import capi

    lib = capi.lib()
    kind = "bf16" if q.dtype == torch.bfloat16 else "f16"
    fn = getattr(lib, f"cta_flash_attention_bwd_{kind}")
    B, nh, T, hs = q.shape
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    s4, s3 = capi.strides(q.stride()), capi.strides(L.stride())
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    delta = torch.empty(B, nh, T, device=q.device)
    nbytes, ws = 0, None
    if stored:
        nbytes = getattr(lib, f"cta_flash_attention_bwd_{kind}_workspace")(B, nh, T, hs,
                                                                            int(causal))
        ws = torch.empty(nbytes // 4 + 4, device=q.device)
    rc = fn(P(q), s4, P(k), s4, P(v), s4, P(O), s4, P(do), s4, P(L), s3, B, nh, T, hs,
            int(causal), P(dq), P(dk), P(dv), P(delta), P(ws) if stored else None, nbytes,
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib.cta_last_error()
    torch.cuda.synchronize()
    return dq, dk, dv


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,nh,T,hs,causal", BWD_SHAPES)
def test_fa2_half_backward_schedules_match_oracle(cuda, bwd_cap, B, nh, T, hs, causal, dtype):
    """Both 16-bit schedules through the C ABI against the float64 oracle with the bounds
    above: stored dS (a workspace) and recompute (none: dK/dV without the dS store, dQ
    recomputing S and dP).  dK and dV are bitwise equal between them (the same kernel body),
    dQ within the 16-bit rounding of a different summation order.  The operator runs the
    recompute schedule at hs 32 and 64 and the stored one at hs 128 (recompute again under a
    workspace cap of 0), with the same bits as the C ABI."""
    from cuda_transformer.ops import flash_attention_bwd, flash_attention_fwd
    from cuda_transformer_amd import _C
    from conftest import rel_err

    q, k, v = _half_inputs(B, nh, T, hs, seed=5000 + T + hs, dtype=dtype)
    do = seeded((B, nh, T, hs), 9000 + T, kind="rand").to(dtype)
    qg, kg, vg, dog = q.to(cuda), k.to(cuda), v.to(cuda), do.to(cuda)
    O, L = flash_attention_fwd(qg, kg, vg, causal)
    stored = _half_bwd_capi(qg, kg, vg, O, dog, L, causal, stored=True)
    recomputed = _half_bwd_capi(qg, kg, vg, O, dog, L, causal, stored=False)
    for grads in (stored, recomputed):
        _bwd_check([g.cpu() for g in grads], q, k, v, do, causal)
    assert torch.equal(recomputed[1], stored[1]) and torch.equal(recomputed[2], stored[2])
    if T > 1:
        assert rel_err(f64(recomputed[0]), f64(stored[0])) <= 4e-3
    op = flash_attention_bwd(qg, kg, vg, O, dog, L, causal)
    torch.cuda.synchronize()
    expect = "stored" if hs == 128 else "recompute"
    assert _C.last_bwd_schedule() == expect
    for a, b in zip(op, stored if expect == "stored" else recomputed):
        assert torch.equal(a, b)
    if hs == 128:
        bwd_cap(0)
        op = flash_attention_bwd(qg, kg, vg, O, dog, L, causal)
        torch.cuda.synchronize()
        assert _C.last_bwd_schedule() == "recompute"
        for a, b in zip(op, recomputed):
            assert torch.equal(a, b)


@pytest.mark.parametrize("schedule", ["stored", "recompute"])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", DTYPES)
def test_fa2_half_config1_as_stated(cuda, dtype, causal, schedule):
    """Benchmark config 1 (B1 H4 N256 D64) with its stated inputs, Q, K, V and dO i.i.d. N(0,1):
    zero-mean dO, where dP - delta cancels most, through both backward schedules."""
    from cuda_transformer.ops import flash_attention_fwd

    q, k, v = _half_inputs(1, 4, 256, 64, seed=123 + int(causal), dtype=dtype)
    do = seeded((1, 4, 256, 64), 129, kind="randn").to(dtype)
    qg, kg, vg = q.to(cuda), k.to(cuda), v.to(cuda)
    O, L = flash_attention_fwd(qg, kg, vg, causal)
    grads = _half_bwd_capi(qg, kg, vg, O, do.to(cuda), L, causal, stored=schedule == "stored")
    _check(O.cpu(), L.cpu(), q, k, v, causal)
    _bwd_check([g.cpu() for g in grads], q, k, v, do, causal)


@pytest.mark.parametrize("schedule", ["recompute", "stored"])
def test_fa2_half_config2_full_size(cuda, schedule):
    """The BF16 path at benchmark config 2's shape (B4 H32 N4096 D64 causal), inputs and dO
    i.i.d. N(0,1), through both backward schedules: two heads against the float64 oracle (the
    forward and gradient bounds above), and on every head the backward's size-independent
    invariants, sum_j dK_j = 0 and sum_j dV_j = sum_i dO_i, within the 16-bit rounding."""
    from cuda_transformer.ops import flash_attention_fwd
    from conftest import rel_err

    B, nh, T, hs = 4, 32, 4096, 64
    print(f"bf16 config 2 full size, {schedule} schedule", flush=True)
    q, k, v = _half_inputs(B, nh, T, hs, seed=2400, dtype=torch.bfloat16)
    do = seeded((B, nh, T, hs), 2404, kind="randn").to(torch.bfloat16)
    qg, kg, vg, dog = q.to(cuda), k.to(cuda), v.to(cuda), do.to(cuda)
    O, L = flash_attention_fwd(qg, kg, vg, True)
    dq, dk, dv = _half_bwd_capi(qg, kg, vg, O, dog, L, True, stored=schedule == "stored")
    for t in (O, L, dq, dk, dv):
        assert torch.isfinite(t).all()
    for b, h in ((0, 0), (B - 1, nh - 1)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        qh, kh, vh, doh = (t[sl] for t in (q, k, v, do))
        _check(O[sl].cpu(), L[sl].cpu(), qh, kh, vh, True)
        O_ref, L_ref = ora.reference_attention(f64(qh), f64(kh), f64(vh), True)
        refs = ora.fa2_backward(f64(qh), f64(kh), f64(vh), O_ref, f64(doh), L_ref, True,
                                br=512, bc=512)
        for got, ref, tol in zip((dq, dk, dv), refs, (3e-2, 3e-2, 1.5e-2)):
            e = rel_err(f64(got[sl].cpu()), ref)
            assert e <= tol, (schedule, b, h, e, tol)
    dk64, dv64, do64 = dk.double(), dv.double(), dog.double()
    assert (dk64.sum(dim=2).abs() <= 1e-2 * dk64.abs().sum(dim=2) + 1e-6).all()
    assert ((dv64.sum(dim=2) - do64.sum(dim=2)).abs() <= 1e-2 * do64.abs().sum(dim=2)).all()
