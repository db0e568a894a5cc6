"""Benchmark + correctness harness: bench, check, log_result.

Mirrors the reference's bench/harness.py:25-91 with two MI355X changes:
  * the cache flush between timed reps reads 1 GiB (the reference zeroes
    256 MiB, :32-33, which does not clear MI355X's 256 MB Infinity Cache on
    top of the 4 MB-per-XCD L2, and a zeroing pass would leave dirty lines
    whose write-back competes with the timed kernel);
  * timestamps are UTC via timezone.utc (Python 3.10 has no datetime.UTC).
"""
from __future__ import annotations

import json
import os
import time
from collections.abc import Callable
from dataclasses import asdict, dataclass
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

import torch
from torch import Tensor

RESULTS_DIR = Path(os.environ.get("RESULTS_DIR", "results"))
FLUSH_BYTES = 1 << 30


@dataclass
class Timing:
    median_ms: float
    p20_ms: float
    p80_ms: float
    mean_ms: float
    n_iters: int


_flush_buf: Tensor | None = None


def flush_caches() -> None:
    """Evict L2 and the Infinity Cache by reading a 1 GiB buffer. A read
    leaves the caches holding clean lines; zeroing the buffer (the
    reference's method) would leave up to the cache capacity of dirty lines
    whose write-back then competes with the timed kernel for HBM."""
    global _flush_buf
    if _flush_buf is None:
        _flush_buf = torch.zeros(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda")
    _flush_buf.max()


def bench(fn: Callable[[], Any], warmup: int = 25, rep: int = 100, flush: bool = True) -> Timing:
    """Time fn() over `rep` calls after `warmup` untimed ones; HIP events on
    the current stream bracket each call (reference bench(), :25-51)."""
    for _ in range(warmup):
        fn()
    if torch.cuda.is_available():
        torch.cuda.synchronize()
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(rep)]
        for start, end in events:
            if flush:
                flush_caches()
            start.record()
            fn()
            end.record()
        torch.cuda.synchronize()
        times = [s.elapsed_time(e) for s, e in events]
    else:
        times = []
        for _ in range(rep):
            t0 = time.perf_counter()
            fn()
            times.append((time.perf_counter() - t0) * 1e3)
    t = torch.tensor(times, dtype=torch.float64)
    p20, p50, p80 = torch.quantile(t, torch.tensor([0.2, 0.5, 0.8], dtype=torch.float64)).tolist()
    return Timing(median_ms=p50, p20_ms=p20, p80_ms=p80, mean_ms=float(t.mean()), n_iters=rep)


@dataclass
class Check:
    passed: bool
    max_abs: float
    max_rel: float
    cosine: float


def check(out: Tensor, ref: Tensor, atol: float = 1e-5, rtol: float = 1e-4) -> Check:
    """Compare in float64; pass iff every |out - ref| <= atol + rtol * |ref|
    (a NaN fails) (reference check(), :62-72)."""
    o = out.detach().double().flatten().cpu()
    r = ref.detach().double().flatten().cpu()
    diff = (o - r).abs()
    return Check(
        passed=bool((diff <= atol + rtol * r.abs()).all()),
        max_abs=diff.max().item(),
        max_rel=(diff / r.abs().clamp_min(1e-12)).max().item(),
        cosine=torch.nn.functional.cosine_similarity(o, r, dim=0).item(),
    )


def log_result(name: str, config: dict, timing: Timing | None = None,
               check: Check | None = None, **metrics: Any) -> None:
    """Append one run (config, timing, check, environment) to
    RESULTS_DIR/<name>.jsonl (reference log_result(), :75-91)."""
    record = {
        "time": datetime.now(timezone.utc).isoformat(timespec="seconds"),
        "config": config,
        "timing": asdict(timing) if timing else None,
        "check": asdict(check) if check else None,
        "env": {
            "gpu": torch.cuda.get_device_name() if torch.cuda.is_available() else "cpu",
            "torch": torch.__version__,
        },
        **metrics,
    }
    RESULTS_DIR.mkdir(parents=True, exist_ok=True)
    with (RESULTS_DIR / f"{name}.jsonl").open("a") as f:
        f.write(json.dumps(record, default=str) + "\n")
