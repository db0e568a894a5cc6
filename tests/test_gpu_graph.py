"""The training step (forward, then backward through bd3_attn_bwd) captured
as one HIP graph: every replay must equal the eager launches bit for bit
(the kernels are deterministic), with unrelated eager work and
synchronisations between the replays. bench.py --graph times the step this way."""
from __future__ import annotations

import pytest
import torch

from _gpu_util import D, bwd_capi, fwd_capi, to_dev, train_inputs
from kernels._native import check, lib, ptr, stream_of, strides


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,n,bs", [(2, 2, 256, 16), (1, 3, 384, 8)])
def test_train_step_graph_replays_match_eager(cuda, B, H, n, bs):
    q, k, v, do = to_dev(train_inputs(B, H, n, seed=7, count=4), cuda)
    o_ref, lse_ref = fwd_capi(q, k, v, bs)
    dq_ref, dk_ref, dv_ref = bwd_capi(q, k, v, o_ref, do, lse_ref, bs)
    torch.cuda.synchronize()

    o = torch.empty_like(q)
    lse = torch.empty_like(lse_ref)
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    nbytes = lib().bd3_attn_bwd_workspace_bytes(B, H, n, D)
    ws = torch.empty(nbytes, device=cuda, dtype=torch.uint8)
    scale = 1.0 / D ** 0.5

    def step():
        s = stream_of(q)  # the current stream: the capture stream while capturing
        check(lib().bd3_attn_fwd(ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), B, H, n, D, bs,
                                 strides(q, k, v, o), scale, s))
        check(lib().bd3_attn_bwd(ptr(q), ptr(k), ptr(v), ptr(o), ptr(do), ptr(lse), ptr(dq), ptr(dk),
                                 ptr(dv), ptr(ws), nbytes, B, H, n, D, bs,
                                 strides(q, k, v, o, do, dq, dk, dv), scale, s))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            step()
    torch.cuda.synchronize()

    for rep in range(3):
        for t in (o, dq, dk, dv):
            t.fill_(float("nan"))
        lse.fill_(float("nan"))
        fwd_capi(k, q, v, bs)  # unrelated eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, want in (("o", o, o_ref), ("lse", lse, lse_ref), ("dq", dq, dq_ref),
                                ("dk", dk, dk_ref), ("dv", dv, dv_ref)):
            assert torch.equal(got, want), (rep, name)
