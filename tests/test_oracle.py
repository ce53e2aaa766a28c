"""Pin the numpy oracle (CPU only).

Every oracle function is checked against (a) the committed golden fixtures, which freeze the
reference's own test oracle (torch CPU math + autograd, float64), (b) closed forms and
invariants fixed by the mathematics, and (c) central finite differences for gradients.
Mutation tests plant plausible mistakes in copies of the oracle (wrong scale, dropped causal
mask, transposed operand, missing delta term, L in log2, a dropped or mis-differentiated
tanh-GELU term) and require that these checks fail.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import attention as ora
from oracle import elementwise as ew
from oracle import linear as lin

GOLDEN = Path(__file__).resolve().parent / "golden"
RNG = np.random.default_rng(1234)


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def d(a):
    return np.asarray(a, dtype=np.float64)


FA2_FIXTURES = ["fa2_b1h1t65d64_causal", "fa2_b1h2t33d32_full", "fa2_b1h1t17d128_causal",
                "fa2_b2h1t24d64_full"]


# ------------------------------------------------------------------ FA2 forward
@pytest.mark.parametrize("name", FA2_FIXTURES)
def test_fa2_forward_matches_golden(name):
    f = load(name)
    causal = bool(f["causal"])
    O, L = ora.fa2_forward(d(f["q"]), d(f["k"]), d(f["v"]), causal)
    np.testing.assert_allclose(O, f["o"], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(L, f["L"], rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("name", FA2_FIXTURES)
def test_fa2_backward_matches_golden(name):
    f = load(name)
    causal = bool(f["causal"])
    O, L = ora.fa2_forward(d(f["q"]), d(f["k"]), d(f["v"]), causal)
    dq, dk, dv = ora.fa2_backward(d(f["q"]), d(f["k"]), d(f["v"]), O, d(f["do"]), L, causal)
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        np.testing.assert_allclose(got, f[key], rtol=1e-9, atol=1e-11)


def _qkv(B, H, T, D, seed=0):
    r = np.random.default_rng(seed)
    return tuple(r.standard_normal((B, H, T, D)) for _ in range(3))


def fwd_closed_form_checks(fwd, T=37, D=16):
    """Closed forms of the forward; returns one bool per check (all True for a correct fwd)."""
    q, k, v = _qkv(2, 2, T, D, seed=1)
    s = 1 / np.sqrt(D)
    out = []
    O, L = fwd(q, k, v, True)
    # causal row 0 only sees key 0
    out.append(np.allclose(O[:, :, 0], v[:, :, 0], atol=1e-12))
    out.append(np.allclose(L[:, :, 0], s * (q[:, :, 0] * k[:, :, 0]).sum(-1), atol=1e-12))
    # the last causal row sees every key: equals the non-causal last row
    On, Ln = fwd(q, k, v, False)
    out.append(np.allclose(O[:, :, -1], On[:, :, -1], atol=1e-12))
    # K = 0, non-causal: uniform weights -> O = mean(V), L = ln T
    Oz, Lz = fwd(q, np.zeros_like(k), v, False)
    out.append(np.allclose(Oz, v.mean(axis=2, keepdims=True) + 0 * Oz, atol=1e-12))
    out.append(np.allclose(Lz, np.log(T), atol=1e-12))
    # constant V rows -> O = that constant
    vc = np.broadcast_to(RNG.standard_normal((1, 1, 1, D)), v.shape).copy()
    Oc, _ = fwd(q, k, vc, True)
    out.append(np.allclose(Oc, vc, atol=1e-12))
    # a single key/query: O = V, L = s q.k
    O1, L1 = fwd(q[:, :, :1], k[:, :, :1], v[:, :, :1], False)
    out.append(np.allclose(O1, v[:, :, :1], atol=1e-12))
    out.append(np.allclose(L1, s * (q[:, :, :1] * k[:, :, :1]).sum(-1), atol=1e-12))
    # non-causal output must depend on future keys (guards against a mask left on)
    out.append(not np.allclose(On[:, :, 0], O[:, :, 0], atol=1e-6))
    # scores are q.k^T, not q.v^T: swapping k and v changes the output for generic inputs
    Os, _ = fwd(q, v, k, False)
    out.append(not np.allclose(Os, On, atol=1e-6))
    # the direct formula agrees (softmax definition, test_flash_attention.py:10-21,32)
    Or, Lr = ora.reference_attention(q, k, v, True)
    out.append(np.allclose(O, Or, atol=1e-12) and np.allclose(L, Lr, atol=1e-12))
    return out


def test_fa2_forward_closed_forms():
    assert all(fwd_closed_form_checks(ora.fa2_forward))


@pytest.mark.parametrize("br,bc", [(16, 16), (7, 5), (64, 3), (1, 1)])
def test_fa2_forward_tile_size_invariance(br, bc):
    q, k, v = _qkv(1, 2, 29, 8, seed=3)
    for causal in (False, True):
        O, L = ora.fa2_forward(q, k, v, causal, br=br, bc=bc)
        Or, Lr = ora.reference_attention(q, k, v, causal)
        np.testing.assert_allclose(O, Or, atol=1e-12)
        np.testing.assert_allclose(L, Lr, atol=1e-12)


def test_fa2_forward_matches_torch_math():
    torch = pytest.importorskip("torch")
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    for (B, H, T, D, causal) in [(1, 3, 50, 32, True), (2, 1, 19, 64, False), (1, 1, 40, 128, True)]:
        q, k, v = _qkv(B, H, T, D, seed=T)
        with sdpa_kernel(SDPBackend.MATH):
            Ot = F.scaled_dot_product_attention(*(torch.from_numpy(t) for t in (q, k, v)),
                                                is_causal=causal, scale=D ** -0.5).numpy()
        O, _ = ora.fa2_forward(q, k, v, causal)
        np.testing.assert_allclose(O, Ot, atol=1e-12)


# ------------------------------------------------------------------ FA2 backward
def _loss_grad_fd(q, k, v, do, causal, which, idx, h=1e-6):
    """Central difference of sum(O * dO) w.r.t. one entry of q, k or v."""
    args = [q.copy(), k.copy(), v.copy()]
    args[which][idx] += h
    lp = (ora.reference_attention(*args, causal)[0] * do).sum()
    args[which][idx] -= 2 * h
    lm = (ora.reference_attention(*args, causal)[0] * do).sum()
    return (lp - lm) / (2 * h)


def bwd_checks(bwd, T=11, D=8):
    """Finite differences + invariants of the backward; one bool per check."""
    q, k, v = _qkv(1, 2, T, D, seed=5)
    do = np.random.default_rng(6).random((1, 2, T, D))
    out = []
    for causal in (True, False):
        O, L = ora.reference_attention(q, k, v, causal)
        g = bwd(q, k, v, O, do, L, causal)
        for which in range(3):
            for idx in [(0, 0, 0, 0), (0, 1, T // 2, D - 1), (0, 1, T - 1, 3)]:
                fd = _loss_grad_fd(q, k, v, do, causal, which, idx)
                out.append(abs(g[which][idx] - fd) <= 1e-6 * max(1.0, abs(fd)))
        dq, dk, dv = g
        out.append(np.allclose(dk.sum(axis=2), 0, atol=1e-12))            # rows of dS sum to 0
        out.append(np.allclose(dv.sum(axis=2), do.sum(axis=2), atol=1e-12))  # rows of P sum to 1
        vc = np.broadcast_to(v[:, :, :1], v.shape).copy()                  # equal V rows
        Oc, Lc = ora.reference_attention(q, k, vc, causal)
        dqc, dkc, _ = bwd(q, k, vc, Oc, do, Lc, causal)
        out.append(np.allclose(dqc, 0, atol=1e-12) and np.allclose(dkc, 0, atol=1e-12))
    return out


def test_fa2_backward_finite_differences_and_invariants():
    assert all(bwd_checks(ora.fa2_backward))


def test_fa2_backward_matches_torch_autograd():
    torch = pytest.importorskip("torch")
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    for (T, D, causal) in [(33, 32, True), (20, 64, False)]:
        q, k, v = _qkv(1, 2, T, D, seed=T + D)
        do = np.random.default_rng(9).random(q.shape)
        tq, tk, tv = (torch.from_numpy(t).requires_grad_() for t in (q, k, v))
        with sdpa_kernel(SDPBackend.MATH):
            o = F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal, scale=D ** -0.5)
        o.backward(torch.from_numpy(do))
        O, L = ora.fa2_forward(q, k, v, causal)
        dq, dk, dv = ora.fa2_backward(q, k, v, O, do, L, causal)
        for got, ref in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
            np.testing.assert_allclose(got, ref.numpy(), atol=1e-11)


def test_fa2_delta_is_rowsum():
    o, do, _ = _qkv(1, 1, 9, 4, seed=8)
    np.testing.assert_allclose(ora.fa2_bwd_delta(o, do), np.einsum("bhtd,bhtd->bht", o, do))


# ------------------------------------------------------------------ mutation tests
def _mutant_scale(q, k, v, causal, br=16, bc=16):
    # softmax scale 1/hs instead of 1/sqrt(hs)
    D = q.shape[-1]
    return ora.fa2_forward(q * np.sqrt(D) / D, k, v, causal, br, bc)


def _mutant_nomask(q, k, v, causal, br=16, bc=16):
    return ora.fa2_forward(q, k, v, False, br, bc)


def _mutant_swap_kv(q, k, v, causal, br=16, bc=16):
    return ora.fa2_forward(q, v, k, causal, br, bc)


def _mutant_log2(q, k, v, causal, br=16, bc=16):
    O, L = ora.fa2_forward(q, k, v, causal, br, bc)
    return O, L / np.log(2.0)


@pytest.mark.parametrize("mutant", [_mutant_scale, _mutant_nomask, _mutant_swap_kv, _mutant_log2])
def test_forward_checks_catch_mutants(mutant):
    assert not all(fwd_closed_form_checks(mutant))


def _bwd_no_delta(q, k, v, o, do, L, causal):
    return ora.fa2_backward(q, k, v, np.zeros_like(o), do, L, causal)


def _bwd_transposed_p(q, k, v, o, do, L, causal):
    # dV from P dO instead of P^T dO (a transposition slip)
    dq, dk, _ = ora.fa2_backward(q, k, v, o, do, L, causal)
    T, D = q.shape[-2], q.shape[-1]
    s = (q @ np.swapaxes(k, -1, -2)) / np.sqrt(D)
    if causal:
        s = np.where(np.triu(np.ones((T, T), bool), 1), -np.inf, s)
    return dq, dk, np.exp(s - L[..., None]) @ do


def _bwd_unscaled_dk(q, k, v, o, do, L, causal):
    dq, dk, dv = ora.fa2_backward(q, k, v, o, do, L, causal)
    return dq, dk * np.sqrt(q.shape[-1]), dv


@pytest.mark.parametrize("mutant", [_bwd_no_delta, _bwd_transposed_p, _bwd_unscaled_dk])
def test_backward_checks_catch_mutants(mutant):
    assert not all(bwd_checks(mutant))


# ------------------------------------------------------------------ linear layer
@pytest.mark.parametrize("name", ["linear_b1t32i65o32", "linear_b2t20i33o48"])
def test_linear_matches_golden(name):
    f = load(name)
    out = lin.fma_forward(d(f["x"]), d(f["w"]), d(f["b"]))
    np.testing.assert_allclose(out, f["out"], rtol=1e-12, atol=1e-12)
    dx, dw, db = lin.linear_backward(d(f["x"]), d(f["w"]), d(f["dy"]))
    np.testing.assert_allclose(dx, f["dx"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dw, f["dw"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(db, f["db"], rtol=1e-12, atol=1e-12)


def test_linear_closed_forms():
    x = RNG.standard_normal((2, 5, 6))
    b = RNG.standard_normal(6)
    np.testing.assert_allclose(lin.fma_forward(x, np.eye(6), b), x + b)
    w = RNG.standard_normal((6, 4))
    # broadcast 2-D weights == explicit batch of identical weights
    np.testing.assert_allclose(lin.fma_forward(x, w, np.zeros(4)),
                               lin.fma_forward(x, np.stack([w, w]), np.zeros(4)))
    # one-hot column selects a column of x
    e = np.zeros((6, 1)); e[3, 0] = 1
    np.testing.assert_allclose(lin.fma_forward(x, e, np.zeros(1))[..., 0], x[..., 3])
    dy = RNG.standard_normal((2, 5, 4))
    np.testing.assert_allclose(lin.db_calculation(dy), dy.sum(axis=(0, 1)))
    # dW by finite differences of sum(out * dy)
    dx, dw, db = lin.linear_backward(x, w, dy)
    h = 1e-6
    for idx in [(0, 0), (5, 3), (2, 1)]:
        wp, wm = w.copy(), w.copy()
        wp[idx] += h
        wm[idx] -= h
        fd = ((lin.fma_forward(x, wp, 0) - lin.fma_forward(x, wm, 0)) * dy).sum() / (2 * h)
        assert abs(dw[idx] - fd) < 1e-6


def test_mlp_matches_torch_autograd_and_finite_differences():
    """fc1 -> GELU -> fc2 composition against torch float64 autograd (F.gelu, erf form) and a
    finite difference through both layers."""
    import torch
    import torch.nn.functional as F

    x = RNG.standard_normal((2, 7, 5))
    w1, b1 = RNG.standard_normal((5, 12)), RNG.standard_normal(12)
    w2, b2 = RNG.standard_normal((12, 5)), RNG.standard_normal(5)
    dz = RNG.standard_normal((2, 7, 5))
    pre, h, out = lin.mlp_forward(x, w1, b1, w2, b2)
    grads = lin.mlp_backward(x, w1, w2, pre, h, dz)
    ts = [torch.tensor(a, requires_grad=True) for a in (x, w1, b1, w2, b2)]
    ref = F.gelu(ts[0] @ ts[1] + ts[2], approximate="none") @ ts[3] + ts[4]
    ref.backward(torch.tensor(dz))
    np.testing.assert_allclose(out, ref.detach().numpy(), rtol=1e-12, atol=1e-12)
    for g, t in zip(grads, ts):
        np.testing.assert_allclose(g, t.grad.numpy(), rtol=1e-11, atol=1e-11)
    eps = 1e-6
    w1p, w1m = w1.copy(), w1.copy()
    w1p[3, 7] += eps
    w1m[3, 7] -= eps
    fd = ((lin.mlp_forward(x, w1p, b1, w2, b2)[2] - lin.mlp_forward(x, w1m, b1, w2, b2)[2])
          * dz).sum() / (2 * eps)
    assert abs(grads[1][3, 7] - fd) < 1e-6


# ------------------------------------------------------------------ GELU
def test_gelu_matches_golden_and_closed_forms():
    f = load("gelu_1x65x32")
    np.testing.assert_allclose(ew.gelu_forward(f["x"]), f["y"], rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(ew.gelu_backward(f["x"], f["dy"]), f["dx"], rtol=1e-12, atol=1e-14)
    assert ew.gelu_forward(0.0) == 0.0
    np.testing.assert_allclose(ew.gelu_forward(1.0), 0.8413447460685429, rtol=1e-15)
    np.testing.assert_allclose(ew.gelu_forward(-1.0), -0.15865525393145707, rtol=1e-14)
    np.testing.assert_allclose(ew.gelu_backward(0.0, 1.0), 0.5, rtol=1e-15)
    x = np.linspace(-5, 5, 41)
    h = 1e-6
    fd = (ew.gelu_forward(x + h) - ew.gelu_forward(x - h)) / (2 * h)
    np.testing.assert_allclose(ew.gelu_backward(x, np.ones_like(x)), fd, atol=1e-8)


def gelu_tanh_checks(fwd, bwd):
    """The tanh-GELU checks as a list of booleans: torch's own float64
    F.gelu(approximate="tanh") and its autograd, the odd-part identity y(x) - y(-x) = x, the
    values at 0, the distance to the erf GELU and finite differences."""
    import torch
    import torch.nn.functional as F

    x = np.concatenate([np.linspace(-12, 12, 481), [-1e4, -30.0, -0.0, 1e-30, 30.0, 1e4]])
    dy = np.random.default_rng(5).standard_normal(x.shape)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    yt = F.gelu(xt, approximate="tanh")
    (dxt,) = torch.autograd.grad(yt, xt, torch.tensor(dy))
    d = np.abs(fwd(x) - ew.gelu_forward(x))
    xs = np.linspace(-6, 6, 49)
    h = 1e-6
    fd = (fwd(xs + h) - fwd(xs - h)) / (2 * h)
    return [
        np.allclose(fwd(x), yt.detach().numpy(), rtol=1e-13, atol=1e-15),
        np.allclose(bwd(x, dy), dxt.numpy(), rtol=1e-12, atol=1e-14),
        np.allclose(fwd(x) - fwd(-x), x, rtol=1e-14, atol=1e-14),
        fwd(0.0) == 0.0 and bwd(0.0, 1.0) == 0.5,
        # the approximation stays within 5e-4 of the erf GELU (its published accuracy)
        1e-5 < d.max() < 5e-4,
        np.allclose(bwd(xs, np.ones_like(xs)), fd, rtol=0, atol=1e-8),
    ]


def test_gelu_tanh_against_torch_and_closed_forms():
    assert all(gelu_tanh_checks(ew.gelu_tanh_forward, ew.gelu_tanh_backward))


def _tanh_gelu(c, k):
    return lambda x: 0.5 * np.asarray(x) * (1.0 + np.tanh(c * (np.asarray(x) + k * np.asarray(x) ** 3)))


def _tanh_gelu_grad(c, k, three=3.0):
    def g(x, dy):
        x = np.asarray(x, dtype=np.float64)
        t = np.tanh(c * (x + k * x**3))
        return dy * (0.5 * (1 + t) + 0.5 * x * (1 - t * t) * c * (1 + three * k * x * x))
    return g


_C, _K = np.sqrt(2 / np.pi), 0.044715


@pytest.mark.parametrize("fwd,bwd", [
    (_tanh_gelu(_C, 0.0), _tanh_gelu_grad(_C, 0.0)),                    # cubic term dropped
    (_tanh_gelu(np.sqrt(np.pi / 2), _K), _tanh_gelu_grad(np.sqrt(np.pi / 2), _K)),  # c inverted
    (_tanh_gelu(_C, _K), _tanh_gelu_grad(_C, _K, three=1.0)),           # d/dx x^3 taken as x^2
    (_tanh_gelu(_C, _K), lambda x, dy: dy * 0.5 * (1 + np.tanh(_C * (x + _K * x**3)))),  # product rule half
])
def test_gelu_tanh_checks_catch_mutants(fwd, bwd):
    assert not all(gelu_tanh_checks(fwd, bwd))


# ------------------------------------------------------------------ softmax
@pytest.mark.parametrize("name", ["softmax_2x9x70", "softmax_1x4x1024"])
def test_softmax_matches_golden(name):
    f = load(name)
    p = ew.softmax_forward(d(f["x"]))
    np.testing.assert_allclose(p, f["p"], rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(ew.softmax_backward(p, d(f["dp"])), f["dx"], rtol=1e-11, atol=1e-14)


def test_softmax_invariants():
    x = RNG.standard_normal((3, 4, 17)) * 3
    p = ew.softmax_forward(x)
    np.testing.assert_allclose(p.sum(-1), 1.0, atol=1e-14)
    np.testing.assert_allclose(ew.softmax_forward(x + 5.0), p, atol=1e-14)
    dp = RNG.standard_normal(x.shape)
    dx = ew.softmax_backward(p, dp)
    np.testing.assert_allclose(dx.sum(-1), 0.0, atol=1e-14)
    h = 1e-6
    xp, xm = x.copy(), x.copy()
    xp[1, 2, 5] += h
    xm[1, 2, 5] -= h
    fd = ((ew.softmax_forward(xp) - ew.softmax_forward(xm)) * dp).sum() / (2 * h)
    np.testing.assert_allclose(dx[1, 2, 5], fd, atol=1e-8)


# ------------------------------------------------------------------ LayerNorm
@pytest.mark.parametrize("name", ["layernorm_9x768", "layernorm_5x65"])
def test_layernorm_matches_golden(name):
    f = load(name)
    y, mean, rstd = ew.layernorm_forward(d(f["x"]), d(f["gamma"]), d(f["beta"]), 1e-5)
    np.testing.assert_allclose(y, f["y"], rtol=1e-12, atol=1e-12)
    dx, dg, db = ew.layernorm_backward(d(f["x"]), d(f["gamma"]), mean, rstd, d(f["dy"]))
    np.testing.assert_allclose(dx, f["dx"], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dg, f["dgamma"], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(db, f["dbeta"], rtol=1e-10, atol=1e-12)


def test_layernorm_invariants():
    x = RNG.standard_normal((6, 50)) * 4 + 2
    g, b = np.ones(50), np.zeros(50)
    y, mean, rstd = ew.layernorm_forward(x, g, b, 1e-5)
    np.testing.assert_allclose(y.mean(-1), 0, atol=1e-12)
    np.testing.assert_allclose(y.var(-1), 1 / (1 + 1e-5 * rstd ** 2), rtol=1e-9)
    dy = RNG.standard_normal(x.shape)
    dx, _, _ = ew.layernorm_backward(x, RNG.standard_normal(50), mean, rstd, dy)
    np.testing.assert_allclose(dx.sum(-1), 0, atol=1e-10)


# ------------------------------------------------------------------ naive attention
@pytest.mark.parametrize("name", ["naive_b1t33h2d32_causal", "naive_b2t17h1d64_full"])
def test_naive_attention_matches_golden(name):
    f = load(name)
    nh, causal = int(f["nh"]), bool(f["causal"])
    qkv = d(f["qkv"])
    out, probs = ora.causal_self_attention_forward(qkv, nh, causal)
    np.testing.assert_allclose(out, f["out"], rtol=1e-11, atol=1e-13)
    np.testing.assert_allclose(probs, f["probs"], rtol=1e-11, atol=1e-14)
    B, T, C3 = qkv.shape
    C = C3 // 3
    hs = C // nh

    def heads(x):
        return x.reshape(B, T, nh, hs).transpose(0, 2, 1, 3).reshape(B * nh, T, hs)

    def unheads(x):
        return x.reshape(B, nh, T, hs).transpose(0, 2, 1, 3).reshape(B, T, C)

    dq, dk, dv = ora.causal_self_attention_backward(
        heads(qkv[..., :C]), heads(qkv[..., C:2 * C]), heads(qkv[..., 2 * C:]),
        probs.reshape(B * nh, T, T), heads(d(f["dO"])))
    s = np.sqrt(hs)  # the op returns dq, dk unscaled; the caller divides by sqrt(hs)
    dqkv = np.concatenate([unheads(dq) / s, unheads(dk) / s, unheads(dv)], -1)
    np.testing.assert_allclose(dqkv, f["dqkv"], rtol=1e-10, atol=1e-12)
