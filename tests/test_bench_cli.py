"""bench.py's contract pieces that need no GPU: the single-GPU guard, the
FLOP convention and the committed traffic figures it reports."""
from __future__ import annotations

import bench


def test_more_than_one_gpu_is_refused(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "ONE GPU" in capsys.readouterr().err


def test_useful_flops_convention():
    # 4 * d * B * H * (n^2 + n * bs): the live pairs of the BD3-LM mask at configs[1]
    assert bench.useful_fwd_flops(8, 12, 1024, 16) == 4 * 64 * 8 * 12 * (1024 * 1024 + 1024 * 16)
    assert bench.useful_fwd_flops(8, 12, 1024, 16) == 26_172_456_960


def test_traffic_figures_are_committed():
    for kernel in ("attn_fwd_dma_kernel", "attn_bwd_delta_kernel", "attn_bwd_kernel", "decode16_partial",
                   "qkv_rope_kernel", "ln_modulate_kernel"):
        t = bench.measured_traffic(kernel)
        assert isinstance(t, int) and t > 0, kernel
    assert bench.measured_traffic("no_such_kernel") is None
