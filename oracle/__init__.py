"""CPU oracle for the BD3-LM attention hot path. TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference's algorithms for the path the
gfx950 kernels implement, so tests can check the kernels against them:

    oracle.mask       the BD3-LM block-diffusion mask and the decode slice
                      (numpy, integer: bit-exact)
    oracle.attention  the eager fp32 masked attention, its autograd
                      gradients, the decode attention and the split-KV
                      LSE merge (torch on the CPU)

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and only as the checker (or, for bench.py, as the timed CPU
baseline). The product path (diffusion-llm_amd/) never imports it and has no
CPU fallback.

Every function cites the reference file:line it follows. How each is pinned
(closed forms, special cases that reduce to library routines, brute force,
finite differences) is in tests/test_oracle_*.py.
"""
