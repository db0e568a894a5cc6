"""The custom ops on the GPU: identical to the direct module calls, and
traceable by torch.compile(dynamic=True, fullgraph=True) with no graph break
(the reference's compile rung), forward, backward and decode."""
from __future__ import annotations

import pytest
import torch

import kernels.ops  # noqa: F401
from kernels.BlockSparseDecodeAttention import block_sparse_decode_attention
from kernels.BlockSparseFlashAttention import BlockSparseFlashAttention
from kernels.SplitKVDecodeAttention import split_kv_decode_attention


def rnd(shape, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dev, torch.bfloat16)


@pytest.mark.gpu
def test_train_op_matches_function(cuda):
    q, k, v, do = (rnd((2, 2, 256, 64), s, cuda) for s in range(4))
    qa, ka, va = (t.clone().requires_grad_() for t in (q, k, v))
    qb, kb, vb = (t.clone().requires_grad_() for t in (q, k, v))
    oa = BlockSparseFlashAttention.apply(qa, ka, va, 16)
    oa.backward(do)
    ob = torch.ops.bd3.attn_fwd(qb, kb, vb, 16)[0]
    ob.backward(do)
    assert torch.equal(oa, ob)
    for a, b in ((qa, qb), (ka, kb), (va, vb)):
        assert torch.equal(a.grad, b.grad)


@pytest.mark.gpu
def test_compile_train_no_graph_break(cuda):
    torch._dynamo.reset()
    q, k, v, do = (rnd((1, 2, 256, 64), s + 10, cuda) for s in range(4))

    def loss(q, k, v):
        return (torch.ops.bd3.attn_fwd(q, k, v, 16)[0].float() * do.float()).sum()

    compiled = torch.compile(loss, backend="aot_eager", fullgraph=True, dynamic=True)
    qe, ke, ve = (t.clone().requires_grad_() for t in (q, k, v))
    qc, kc, vc = (t.clone().requires_grad_() for t in (q, k, v))
    le = loss(qe, ke, ve)
    le.backward()
    lc = compiled(qc, kc, vc)
    lc.backward()
    assert torch.equal(le, lc)
    for a, b in ((qe, qc), (ke, kc), (ve, vc)):
        assert torch.equal(a.grad, b.grad)


@pytest.mark.gpu
def test_compile_decode_no_graph_break(cuda):
    torch._dynamo.reset()
    q, k, v = rnd((2, 3, 16, 64), 20, cuda), rnd((2, 3, 272, 64), 21, cuda), rnd((2, 3, 272, 64), 22, cuda)
    f = torch.compile(lambda q, k, v: torch.ops.bd3.decode(q, k, v, 16, 0) * 2, backend="aot_eager",
                      fullgraph=True, dynamic=True)
    assert torch.equal(f(q, k, v), block_sparse_decode_attention(q, k, v, 16) * 2)
    g = torch.compile(lambda q, k, v: torch.ops.bd3.decode(q, k, v, 16, -1), backend="aot_eager",
                      fullgraph=True, dynamic=True)
    assert torch.equal(g(q, k, v), split_kv_decode_attention(q, k, v, 16))
    # a second shape reuses the dynamic graph
    k2, v2 = rnd((2, 3, 400, 64), 23, cuda), rnd((2, 3, 400, 64), 24, cuda)
    assert torch.equal(f(q, k2, v2), block_sparse_decode_attention(q, k2, v2, 16) * 2)
