"""bd3_clock_probe (the benchmark's shader-clock measurement) on the GPU:
every workgroup reports positive tick counts and the clock they imply lies
in the range an MI355X can run at (its engine clock peaks at 2.4 GHz)."""
import ctypes

import pytest
import torch

from kernels._native import lib
from perf.harness import shader_clock_ghz

pytestmark = pytest.mark.gpu


def test_clock_probe_ticks_and_range():
    dev = torch.device("cuda:0")
    wgs = 300
    out = torch.zeros(2 * wgs, dtype=torch.int64, device=dev)
    rate = ctypes.c_int64(0)
    assert lib().bd3_clock_probe(ctypes.c_void_p(out.data_ptr()), wgs, 2000, ctypes.byref(rate), None) == 0
    torch.cuda.synchronize()
    t = out.view(wgs, 2).cpu()
    assert rate.value > 0
    assert bool((t > 0).all()), "every workgroup writes its two tick counts"
    r = shader_clock_ghz(lib(), dev, workgroups=512, iters=4000)
    print(f"shader clock under MFMA load: {r['median']:.3f} GHz (min {r['min']:.3f}, max {r['max']:.3f})")
    assert 0.3 < r["min"] <= r["median"] <= r["max"] < 2.6
