"""The torch.library custom ops (kernels/ops.py) on a machine without a GPU:
registered under torch.ops.bd3, and their fake kernels give the real
kernels' output shapes and dtypes (what torch.compile traces with)."""
from __future__ import annotations

import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import kernels.ops  # noqa: F401


def test_ops_registered():
    for name in ("attn_fwd", "attn_bwd", "decode"):
        assert hasattr(torch.ops.bd3, name)


def test_fake_shapes():
    with FakeTensorMode():
        q, k, v = (torch.empty(2, 3, 256, 64, dtype=torch.bfloat16) for _ in range(3))
        o, lse = torch.ops.bd3.attn_fwd(q, k, v, 16)
        assert o.shape == q.shape and o.dtype == torch.bfloat16
        assert lse.shape == (2, 3, 256) and lse.dtype == torch.float32
        dq, dk, dv = torch.ops.bd3.attn_bwd(q, k, v, o, lse, o, 16)
        assert dq.shape == dk.shape == dv.shape == q.shape
        qd = torch.empty(2, 3, 16, 64, dtype=torch.bfloat16)
        kd = torch.empty(2, 3, 300, 64, dtype=torch.bfloat16)
        od = torch.ops.bd3.decode(qd, kd, kd, 16, 0)
        assert od.shape == qd.shape and od.dtype == torch.bfloat16
