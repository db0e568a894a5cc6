"""Device timing for the benchmarks: per-call HIP-event samples taken on the
launch stream, each call preceded by an eviction of the GPU caches.

The events are created with hipEventDisableSystemFence (`StreamEvent`). A
default HIP timing event writes back and invalidates the GPU caches when it
is recorded; on MI355X that adds several microseconds to every timed interval
(measured: the three training kernels' event times exceed their rocprofv3
kernel durations by 5-6 us each) and empties the caches the next kernel
would have found warm. The fence-free event only stamps the time.

The reference times its kernels with CUDA events after clearing a 256 MiB
buffer (bench/harness.py:25-51). On MI355X that does not empty the caches a
kernel's inputs may sit in: 4 MB of L2 per XCD plus the 256 MB Infinity
Cache in front of HBM. `CacheEvictor` therefore streams a 1 GiB buffer
through them with a read (a reduction), which leaves clean lines behind; a
zeroing pass would leave dirty lines whose write-back would then compete
with the timed call for HBM.

    samples = time_calls(fn, reps=30, warmup=5)   # flush, event, fn(), event
    samples.median_ms, samples.quantile_ms(0.2), samples.mean_ms

Results are kept as the reference keeps them (bench/harness.py:62-91):
`check(out, ref)` compares in float64 (pass iff |out - ref| <= atol + rtol *
|ref| everywhere) and `log_result(name, config, timing, check, **metrics)`
appends one JSON record per run to RESULTS_DIR/<name>.jsonl.
"""
from __future__ import annotations

import ctypes
import json
import os
import statistics
import time
from collections.abc import Callable, Sequence
from dataclasses import asdict, dataclass
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

import torch

EVICT_BYTES = 1 << 30
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hip_runtime_api.h

_hip: ctypes.CDLL | None = None


def _hip_runtime() -> ctypes.CDLL:
    """The HIP runtime torch has loaded (found by its soname), with the
    event entry points typed."""
    global _hip
    if _hip is None:
        torch.cuda.init()
        h = None
        for soname in ("libamdhip64.so.7", "libamdhip64.so"):
            try:
                h = ctypes.CDLL(soname)
                break
            except OSError:
                continue
        if h is None:
            raise RuntimeError("the HIP runtime (libamdhip64) is not loadable")
        vp, p = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
        h.hipEventCreateWithFlags.argtypes = [p, ctypes.c_uint]
        h.hipEventRecord.argtypes = [vp, vp]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        h.hipEventDestroy.argtypes = [vp]
        for f in (h.hipEventCreateWithFlags, h.hipEventRecord, h.hipEventElapsedTime, h.hipEventDestroy):
            f.restype = ctypes.c_int
        _hip = h
    return _hip


class StreamEvent:
    """A HIP timing event without the system-scope fence (see the module
    docstring), recorded on a torch stream."""

    def __init__(self):
        self._h = _hip_runtime()
        self._ev = ctypes.c_void_p()
        st = self._h.hipEventCreateWithFlags(ctypes.byref(self._ev), HIP_EVENT_DISABLE_SYSTEM_FENCE)
        if st != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed: {st}")

    def record(self, stream: torch.cuda.Stream | None = None) -> None:
        stream = stream or torch.cuda.current_stream()
        st = self._h.hipEventRecord(self._ev, ctypes.c_void_p(stream.cuda_stream))
        if st != 0:
            raise RuntimeError(f"hipEventRecord failed: {st}")

    def elapsed_time(self, end: "StreamEvent") -> float:
        """Milliseconds from this event to `end` (both must have completed)."""
        ms = ctypes.c_float()
        st = self._h.hipEventElapsedTime(ctypes.byref(ms), self._ev, end._ev)
        if st != 0:
            raise RuntimeError(f"hipEventElapsedTime failed: {st}")
        return ms.value

    def __del__(self):
        if getattr(self, "_ev", None) and self._ev.value:
            self._h.hipEventDestroy(self._ev)
            self._ev = ctypes.c_void_p()


class CacheEvictor:
    """Owns the eviction buffer (allocated on first use, on the current
    device) and reads it through the caches on `evict()`."""

    def __init__(self, nbytes: int = EVICT_BYTES):
        self.nbytes = nbytes
        self._buf: torch.Tensor | None = None

    def evict(self) -> None:
        if self._buf is None:
            self._buf = torch.ones(self.nbytes // 4, dtype=torch.int32, device="cuda")
        self._buf.max()


_EVICTOR = CacheEvictor()


def flush_caches() -> None:
    """Evict L2 and the Infinity Cache with the shared 1 GiB read."""
    _EVICTOR.evict()


class Samples:
    """Per-call durations in milliseconds, with the summary statistics the
    bench records report."""

    def __init__(self, ms: Sequence[float]):
        if not ms:
            raise ValueError("no samples")
        self.ms = sorted(float(x) for x in ms)

    def quantile_ms(self, p: float) -> float:
        """Linear-interpolated quantile, 0 <= p <= 1."""
        pos = p * (len(self.ms) - 1)
        lo = int(pos)
        hi = min(lo + 1, len(self.ms) - 1)
        return self.ms[lo] + (self.ms[hi] - self.ms[lo]) * (pos - lo)

    @property
    def median_ms(self) -> float:
        return self.quantile_ms(0.5)

    @property
    def p20_ms(self) -> float:
        return self.quantile_ms(0.2)

    @property
    def p80_ms(self) -> float:
        return self.quantile_ms(0.8)

    @property
    def mean_ms(self) -> float:
        return statistics.fmean(self.ms)

    @property
    def n_iters(self) -> int:
        return len(self.ms)


def time_calls(fn: Callable[[], Any], reps: int = 30, warmup: int = 5, flush: bool = True,
               stream: torch.cuda.Stream | None = None) -> Samples:
    """Run fn() `warmup` times untimed, then `reps` times, each timed by a
    pair of StreamEvents recorded on `stream` (default: the current stream,
    which is where the library's wrappers launch). With `flush`, the caches
    are evicted before every timed call, outside the events. Without a GPU
    the host clock times each call instead."""
    for _ in range(warmup):
        fn()
    if not torch.cuda.is_available():
        ms = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ms.append((time.perf_counter() - t0) * 1e3)
        return Samples(ms)
    stream = stream or torch.cuda.current_stream()
    torch.cuda.synchronize()
    marks = []
    for _ in range(reps):
        if flush:
            flush_caches()
        start, stop = StreamEvent(), StreamEvent()
        start.record(stream)
        fn()
        stop.record(stream)
        marks.append((start, stop))
    torch.cuda.synchronize()
    return Samples([a.elapsed_time(b) for a, b in marks])


def bench(fn: Callable[[], Any], warmup: int = 5, rep: int = 30, flush: bool = True) -> Samples:
    """time_calls with the argument names the bench sections use."""
    return time_calls(fn, reps=rep, warmup=warmup, flush=flush)


def shader_clock_ghz(lib: ctypes.CDLL, device: torch.device, workgroups: int = 1024,
                     iters: int = 40000) -> dict:
    """The shader clock the chip holds under a full matrix-core load, from
    `bd3_clock_probe` (every SIMD busy with independent bf16 MFMA chains for
    ~10 ms): per workgroup, shader-clock ticks over constant-rate real-time
    ticks times the real-time rate. Returns the median and extremes over the
    workgroups in GHz, and the bf16 dense peak that clock gives (256 CUs x
    4096 FLOP per clock)."""
    out = torch.zeros(2 * workgroups, dtype=torch.int64, device=device)
    rate = ctypes.c_int64(0)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    for _ in range(2):  # the first launch settles the clock; the second is read
        rc = lib.bd3_clock_probe(ctypes.c_void_p(out.data_ptr()), workgroups, iters, ctypes.byref(rate), stream)
        if rc != 0:
            raise RuntimeError(f"bd3_clock_probe failed: {lib.bd3_last_error().decode()}")
    torch.cuda.synchronize(device)
    t = out.view(workgroups, 2).double().cpu()
    ghz = (t[:, 0] / t[:, 1] * rate.value / 1e6).tolist()
    ghz.sort()
    med = ghz[len(ghz) // 2]
    return {"median": med, "min": ghz[0], "max": ghz[-1], "wall_rate_khz": rate.value,
            "bf16_peak_tflops": 256 * 4096 * med * 1e9 / 1e12,
            "probe": f"{workgroups} workgroups x 4 waves, {iters} rounds of 4 independent 32x32x16 bf16 MFMAs"}


RESULTS_DIR = Path(os.environ.get("RESULTS_DIR", "results"))


@dataclass
class Check:
    """Outcome of `check`: pass / fail plus the float64 error figures."""
    passed: bool
    max_abs: float
    max_rel: float
    cosine: float


def check(out: torch.Tensor, ref: torch.Tensor, atol: float = 1e-5, rtol: float = 1e-4) -> Check:
    """Element-wise comparison in float64: passes iff every |out - ref| <=
    atol + rtol * |ref| (a NaN anywhere fails). max_rel divides by |ref|
    clamped at 1e-12 and is informational (it grows where ref ~ 0)."""
    o = out.detach().to("cpu", torch.float64).reshape(-1)
    r = ref.detach().to("cpu", torch.float64).reshape(-1)
    if o.shape != r.shape:
        raise ValueError(f"shape mismatch: {tuple(out.shape)} vs {tuple(ref.shape)}")
    diff = (o - r).abs()
    ok = bool(torch.all(diff <= atol + rtol * r.abs()))  # NaN compares false
    den = float(o.norm() * r.norm())
    return Check(passed=ok,
                 max_abs=float(diff.max()) if diff.numel() else 0.0,
                 max_rel=float((diff / r.abs().clamp_min(1e-12)).max()) if diff.numel() else 0.0,
                 cosine=float(torch.dot(o, r)) / den if den > 0 else float("nan"))


def _timing_record(timing: Any) -> dict | None:
    if timing is None:
        return None
    if isinstance(timing, Samples):
        return {"median_ms": timing.median_ms, "p20_ms": timing.p20_ms, "p80_ms": timing.p80_ms,
                "mean_ms": timing.mean_ms, "n_iters": timing.n_iters}
    if isinstance(timing, dict):
        return timing
    return asdict(timing)


def _environment() -> dict:
    env = {"torch": torch.__version__, "hip": getattr(torch.version, "hip", None)}
    if torch.cuda.is_available():
        env["gpu"] = torch.cuda.get_device_name()
        props = torch.cuda.get_device_properties(torch.cuda.current_device())
        env["gcn_arch"] = getattr(props, "gcnArchName", None)
        env["compute_units"] = props.multi_processor_count
    else:
        env["gpu"] = "cpu"
    try:
        from kernels._native import LIB_PATH, lib
        if LIB_PATH.exists():
            env["bd3_abi_version"] = lib().bd3_abi_version()
    except Exception:  # the record is still useful without the library
        pass
    return env


def log_result(name: str, config: dict, timing: Any = None, check: Check | None = None, **metrics: Any) -> Path:
    """Append one run to RESULTS_DIR/<name>.jsonl: UTC time, the config, the
    timing (a Samples, a dict or a dataclass), the check, the environment
    (GPU, torch / HIP versions, library ABI) and any extra metrics. Returns
    the file written."""
    record = {
        "time": datetime.now(timezone.utc).isoformat(timespec="seconds"),
        "config": config,
        "timing": _timing_record(timing),
        "check": asdict(check) if check is not None else None,
        "env": _environment(),
        **metrics,
    }
    RESULTS_DIR.mkdir(parents=True, exist_ok=True)
    path = RESULTS_DIR / f"{name}.jsonl"
    with path.open("a") as f:
        f.write(json.dumps(record, default=str) + "\n")
    return path
