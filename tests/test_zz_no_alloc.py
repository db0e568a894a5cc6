"""bd3_attn_bwd_noalloc (the backward without a caller workspace) against
bd3_attn_bwd: the same kernels, so dQ, dK, dV must be bit-identical; two
calls in a row, the second smaller, so a stale scratch array from the first
call would show."""
import ctypes

import pytest
import torch

from _gpu_util import D, bwd_capi, fwd_capi, to_dev, train_inputs
from kernels import _native
from kernels._native import check, lib, ptr, stream_of, strides


def bwd_noalloc(q, k, v, o, dout, lse, block_size):
    B, H, S, _ = q.shape
    dq, dk, dv = (torch.full_like(q, float("nan")) for _ in range(3))
    check(lib().bd3_attn_bwd_noalloc(ptr(q), ptr(k), ptr(v), ptr(o), ptr(dout), ptr(lse), ptr(dq), ptr(dk),
                                     ptr(dv), B, H, S // 2, D, block_size,
                                     strides(q, k, v, o, dout, dq, dk, dv), 1.0 / D ** 0.5, stream_of(q)))
    return dq, dk, dv


@pytest.mark.gpu
def test_noalloc_backward_equals_workspace_backward(cuda):
    for B, H, n, bs in ((4, 12, 1024, 16), (1, 3, 256, 4)):  # the second call is smaller
        print(f"bwd_noalloc B={B} H={H} n={n} bs={bs}", flush=True)
        q, k, v, do = to_dev(train_inputs(B, H, n, seed=n + bs, count=4), cuda)
        o, lse = fwd_capi(q, k, v, bs)
        want = bwd_capi(q, k, v, o, do, lse, bs)
        got = bwd_noalloc(q, k, v, o, do, lse, bs)
        torch.cuda.synchronize()
        for name, a, b in zip(("dq", "dk", "dv"), got, want):
            assert torch.equal(a, b), f"{name} differs at B={B} H={H} n={n} bs={bs}"


def test_noalloc_rejects_rows_beyond_its_array():
    """batch * heads * 2n above BD3_NOALLOC_MAX_ROWS (2^20) is refused before
    any device call."""
    st = (ctypes.c_int64 * 24)(*([64 * 4096, 64 * 4096, 64] * 8))
    fake = 0x100000
    status = _native.lib().bd3_attn_bwd_noalloc(*[fake] * 9, 8, 16, 4096 + 128, 64, 16, st, 0.125, None)
    assert status == _native.BD3_EINVAL
    assert "at most 1048576 rows" in _native.last_error()


@pytest.mark.gpu
def test_noalloc_backward_replays_from_a_graph(cuda):
    """Callers under HIP graph capture: after one eager call on the device
    (which looks up the scratch array's address), the entry point is
    captured into a graph; three replays, each after the outputs are
    poisoned by eager work, equal bd3_attn_bwd bit for bit."""
    B, H, n, bs = 2, 4, 512, 16
    print(f"bwd_noalloc graph B={B} H={H} n={n} bs={bs}", flush=True)
    q, k, v, do = to_dev(train_inputs(B, H, n, seed=7, count=4), cuda)
    o, lse = fwd_capi(q, k, v, bs)
    want = bwd_capi(q, k, v, o, do, lse, bs)
    dq, dk, dv = (torch.full_like(q, float("nan")) for _ in range(3))
    st = strides(q, k, v, o, do, dq, dk, dv)

    def call():
        check(lib().bd3_attn_bwd_noalloc(ptr(q), ptr(k), ptr(v), ptr(o), ptr(do), ptr(lse), ptr(dq), ptr(dk),
                                         ptr(dv), B, H, n, D, bs, st, 1.0 / D ** 0.5,
                                         torch.cuda.current_stream().cuda_stream))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()  # eager warm-up on the device
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    torch.cuda.synchronize()
    for rep in range(3):
        for t in (dq, dk, dv):
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
            assert torch.equal(a, b), f"{name} differs at replay {rep}"
