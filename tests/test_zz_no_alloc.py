"""The allocation-free backward entry point against the backward it is a variant of.

cta_flash_attention_bwd_noalloc keeps delta in the library's own device array instead of caller
scratch and runs the reference's schedule, so its gradients must be bitwise equal to
cta_flash_attention_bwd called with caller-provided delta and no dS workspace.  Two calls in a
row, the second on a smaller problem (the array keeps the first call's contents), each compared
bitwise, plus a check against the float64 oracle at the suite's tolerances.  The size limit is
checked on the host, before any launch.
"""
import re

import numpy as np
import pytest
import torch

from conftest import assert_rel_err, f64, seeded
from oracle import attention as ora

pytestmark = pytest.mark.gpu

CASES = [(2, 4, 300, 64, True), (1, 2, 97, 32, False)]  # second call: smaller input


def _inputs(B, nh, T, hs, seed, cuda):
    q, k, v = (seeded((B, nh, T, hs), seed + i).to(cuda) for i in range(3))
    do = seeded((B, nh, T, hs), seed + 3, kind="rand").to(cuda)
    return q, k, v, do


def _bwd(capi, name, q, k, v, O, do, L, causal, with_scratch):
    B, nh, T, hs = q.shape
    s4, s3 = capi.strides(q.stride()), capi.strides(L.stride())
    st = torch.cuda.current_stream().cuda_stream
    grads = [torch.full_like(q, float("nan")) for _ in range(3)]
    args = [q.data_ptr(), s4, k.data_ptr(), s4, v.data_ptr(), s4, O.data_ptr(), s4,
            do.data_ptr(), s4, L.data_ptr(), s3, B, nh, T, hs, int(causal),
            *(g.data_ptr() for g in grads)]
    if with_scratch:
        delta = torch.empty(B, nh, T, device=q.device)
        args += [delta.data_ptr(), None, 0]
    capi.call(name, *args, st)
    torch.cuda.synchronize()
    return grads


def test_noalloc_bwd_matches_bwd_twice(cuda):
    from cuda_transformer.ops import flash_attention_fwd
    from cuda_transformer_amd import capi

    for i, (B, nh, T, hs, causal) in enumerate(CASES):
        print(f"noalloc call {i}: B{B} H{nh} T{T} D{hs} causal={causal}", flush=True)
        q, k, v, do = _inputs(B, nh, T, hs, 500 + 10 * i, cuda)
        O, L = flash_attention_fwd(q, k, v, causal)
        got = _bwd(capi, "cta_flash_attention_bwd_noalloc", q, k, v, O, do, L, causal, False)
        ref = _bwd(capi, "cta_flash_attention_bwd", q, k, v, O, do, L, causal, True)
        for g, r in zip(got, ref):
            assert torch.equal(g, r)
        refs = ora.fa2_backward(f64(q), f64(k), f64(v), f64(O), f64(do), f64(L), causal,
                                br=64, bc=64)
        for g, r in zip(got, refs):
            np.testing.assert_allclose(f64(g), r, rtol=1e-5, atol=1e-4)
            assert_rel_err(f64(g), r, 1e-3)


def test_noalloc_bwd_in_a_hip_graph(cuda):
    """One allocation-free backward captured in a HIP graph, after an eager call has resolved the
    library's device array on this device, then replayed twice with eager work between the
    replays: every replay equals the eager result bit for bit."""
    from cuda_transformer.ops import flash_attention_fwd
    from cuda_transformer_amd import capi

    B, nh, T, hs, causal = 2, 4, 300, 64, True
    q, k, v, do = _inputs(B, nh, T, hs, 700, cuda)
    O, L = flash_attention_fwd(q, k, v, causal)
    s4, s3 = capi.strides(q.stride()), capi.strides(L.stride())
    grads = [torch.empty_like(q) for _ in range(3)]

    def call():
        capi.call("cta_flash_attention_bwd_noalloc", q.data_ptr(), s4, k.data_ptr(), s4,
                  v.data_ptr(), s4, O.data_ptr(), s4, do.data_ptr(), s4, L.data_ptr(), s3, B, nh,
                  T, hs, int(causal), *(g.data_ptr() for g in grads),
                  torch.cuda.current_stream().cuda_stream)

    call()
    torch.cuda.synchronize()
    eager = [g.clone() for g in grads]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for rep in range(2):
        for g in grads:
            g.fill_(float("nan"))
        flash_attention_fwd(q, k, v, causal)  # eager work between the replays
        graph.replay()
        torch.cuda.synchronize()
        for g, e in zip(grads, eager):
            assert torch.equal(g, e), f"replay {rep} differs from the eager call"


def test_noalloc_bwd_rejects_too_many_rows(cuda):
    from cuda_transformer_amd import capi

    B, nh, hs = 1, 1, 64
    T = int(re.search(r"#define CTA_BWD_NOALLOC_MAX_ROWS (\d+)", capi.HEADER.read_text()).group(1))
    s4 = capi.strides((0, 0, hs, 1))
    s3 = capi.strides((0, 0, 1))
    # Pointers are never dereferenced: the size check fails before anything is launched.
    x = torch.empty(16, device=cuda)
    p = x.data_ptr()
    with pytest.raises(capi.CtaError, match="exceeds the allocation-free scratch"):
        capi.call("cta_flash_attention_bwd_noalloc", p, s4, p, s4, p, s4, p, s4, p, s4, p, s3,
                  B, nh, T + 1, hs, 1, p, p, p, torch.cuda.current_stream().cuda_stream)
