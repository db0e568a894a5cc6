"""Measurement support for the BD3-LM attention kernels (the counterpart of
the reference's bench/harness.py and bench/attention_bench.py conventions)."""
