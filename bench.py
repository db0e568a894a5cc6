#!/usr/bin/env python3
"""Benchmark of the BD3-LM attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Headline: one step = BD3-LM training attention
forward + backward (bd3_attn_fwd, then the backward's Delta pass
bd3_attn_bwd_delta and its main launch bd3_attn_bwd_main, through the C ABI,
launched one after the other on one stream; --graph replays them from
captured HIP graphs instead) at
B=8, L=1024 (sequence 2048), H=12, d=64, block 16, bf16, q/k/v/dO ~ N(0,1)
from seed 0, resident in HBM. value = useful fwd+bwd FLOPs per second:
3.5 x 4*d*B*H*(n^2 + n*bs) (the reference's convention,
bench/attention_bench.py:89,99, restricted to unmasked pairs).

Printed on stdout as ONE JSON line, with:
  roofline      the dominant kernel's useful TFLOP/s against bf16 dense MFMA
                peak (the mean of HIP-event spans around that launch over K
                steps of the same protocol); traffic = its HBM bytes per launch from the committed
                rocprofv3 FETCH_SIZE / WRITE_SIZE summary
                (profiles/hbm_traffic_pmc.md);
  cpu_baseline  the fp32 eager oracle's fwd+bwd (and fwd alone) on the host
                cores over a bounded sample of (b, h) slices of the same
                workload; the decode section carries the eager decode
                oracle's K+V GB/s on the host the same way;
  decode        configs[3]: split-KV decode KV-read GB/s at splits
                {1, 4, 8, 16}, the reference's default split rule and the
                auto split, against 8 TB/s;
  kv_cache      the layer's attention inputs (split + RoPE + cache
                placement, bd3_qkv_rope) at configs[3]'s decode step and a
                full 8 x 2048-token sequence, against the reference's eager
                path (RoPE as bf16 ops + torch.cat of the cache);
  sampling      one denoising step's SUBS + Gumbel-max draw
                (bd3_subs_sample) at configs[4]'s and configs[3]'s step
                shapes against the reference's eager float64 path;
  dit_glue      LayerNorm + adaLN modulate and the gated residual
                (bd3_ln_modulate, bd3_gate_residual) at configs[1]'s and
                configs[4]'s shapes against the reference's eager ops;
  e2e           configs[4]: the restated BD3-LM sampler (8 x 2048 tokens,
                blocks of 32, 32 steps) with this library on the attention
                path: tokens/s, the eager path's tokens/s on its first
                blocks, logit max-abs vs the eager backbone;
  sweep         configs[2]: block sizes {4, 16, 64, 256} at B=4, L=2048,
                H=16 (useful TFLOP/s and the schedule's useful fraction).
Human-readable progress goes to stderr.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (str(REPO), str(REPO / "diffusion-llm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
D = 64


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def useful_fwd_flops(B, H, n, bs):
    return 4 * D * B * H * (n * n + n * bs)


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (profiles/hbm_traffic_pmc.md, calibrated
    against a copy of known size), or None if it is not there."""
    path = REPO / "profiles" / "hbm_traffic_pmc.md"
    try:
        for line in path.read_text().splitlines():
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic" and parts[1] == kernel:
                return int(parts[2])
    except OSError:
        pass
    return None


def seeded_bf16(shape, seed, count, device):
    import torch
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g, dtype=torch.float32).to(device, torch.bfloat16)
            for _ in range(count)]


class TrainStep:
    """Preallocated forward + backward of the training attention via the C ABI."""

    def __init__(self, B, H, n, bs, device, seed=0):
        import torch
        from kernels._native import lib, ptr, stream_of, strides
        self.B, self.H, self.n, self.bs = B, H, n, bs
        self.q, self.k, self.v, self.do = seeded_bf16((B, H, 2 * n, D), seed, 4, device)
        self.o = torch.empty_like(self.q)
        self.lse = torch.empty((B, H, 2 * n), device=device, dtype=torch.float32)
        self.dq, self.dk, self.dv = (torch.empty_like(self.q) for _ in range(3))
        self.delta = torch.empty((2, B, H, 2 * n), device=device, dtype=torch.float32)  # Delta, -L / scale
        self.lib = lib()
        self.fwd_strides = strides(self.q, self.k, self.v, self.o)
        self.delta_strides = strides(self.o, self.do)
        self.main_strides = strides(self.q, self.k, self.v, self.do, self.dq, self.dk, self.dv)
        self.stream = stream_of(self.q)
        self.p = {name: ptr(getattr(self, name)) for name in
                  ("q", "k", "v", "o", "lse", "do", "dq", "dk", "dv", "delta")}
        self.scale = 1.0 / D ** 0.5

    def fwd(self):
        from kernels._native import check
        p = self.p
        check(self.lib.bd3_attn_fwd(p["q"], p["k"], p["v"], p["o"], p["lse"], self.B, self.H, self.n, D,
                                    self.bs, self.fwd_strides, self.scale, self.stream))

    def bwd_delta(self):
        """bd3_attn_bwd_delta: Delta and -L / scale (the backward's first launch)."""
        from kernels._native import check
        p = self.p
        check(self.lib.bd3_attn_bwd_delta(p["o"], p["do"], p["lse"], p["delta"], self.B, self.H, self.n, D, self.bs,
                                          self.delta_strides, self.scale, self.stream))

    def bwd_main(self):
        """bd3_attn_bwd_main: every dQ and dK/dV item in one launch."""
        from kernels._native import check
        p = self.p
        check(self.lib.bd3_attn_bwd_main(p["q"], p["k"], p["v"], p["do"], p["lse"], p["delta"], p["dq"], p["dk"],
                                         p["dv"], self.B, self.H, self.n, D, self.bs, self.main_strides, self.scale,
                                         self.stream))

    def bwd(self):
        """bd3_attn_bwd's two launches."""
        self.bwd_delta()
        self.bwd_main()

    def useful_flops(self):
        return 3.5 * useful_fwd_flops(self.B, self.H, self.n, self.bs)


def _capture_step(step: TrainStep):
    """The forward and the backward (dQ + dK/dV launches) captured as two HIP
    graphs on a side stream. Returns (forward replay, backward replay), or
    None when capture is not available; the caller then launches the kernels
    eagerly."""
    import torch
    saved = step.stream
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graphs = (torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph())
        with torch.cuda.stream(side):
            step.stream = torch.cuda.current_stream().cuda_stream
            step.fwd()
            step.bwd()
            torch.cuda.synchronize()
            with torch.cuda.graph(graphs[0], stream=side):
                step.fwd()
            with torch.cuda.graph(graphs[1], stream=side):
                step.bwd()
        step.stream = saved
        torch.cuda.synchronize()
        return graphs[0].replay, graphs[1].replay
    except Exception as exc:  # capture unsupported: eager launches
        log(f"graph capture unavailable ({exc}); timing eager launches")
        step.stream = saved
        torch.cuda.synchronize()
        return None


def time_train(step: TrainStep, steps: int, warmup: int, use_graph: bool = False, ramp_s: float = 2.0):
    """Ramp the clocks (eager steps for ramp_s seconds), run `warmup`
    untimed steps, then time exactly `steps` fwd+bwd steps between two
    synchronisations, in the reference microbench's protocol
    (bench/attention_bench.py:61-76 with bench/harness.py:25-51): the caches
    are evicted (a 1 GiB read, larger than the 256 MB Infinity Cache) before
    the forward and again before the backward, and HIP events on the launch
    stream (fence-free, perf.harness.StreamEvent) time each; fwd+bwd is their
    sum. As in the reference, one pair of events brackets the whole backward
    (an event between its two launches adds ~1.3 us of dispatch gap); the
    split between the Delta pass and the main launch comes from `steps` more
    steps of the same protocol with an event between them. With `use_graph`
    the forward and the backward are replayed from two captured HIP graphs.
    The same steps are also timed back to back without eviction (wall clock)
    for comparison.

    Returns a dict: step_ms (median, p20, p80, mean of fwd + bwd over the
    timed steps), kernel_ms / kernel_mean_ms (median / mean of each kernel),
    warm_ms_per_step, launch."""
    import torch
    from perf.harness import Samples, StreamEvent, flush_caches
    # Ramp: on a freshly started process the step runs ~15% slow for the
    # first ~1.5 s of load (clocks and first touches settling), far longer
    # than W warm-up steps last.
    t_end = time.perf_counter() + ramp_s
    while time.perf_counter() < t_end:
        for _ in range(20):
            step.fwd()
            step.bwd()
        torch.cuda.synchronize()
    for _ in range(warmup):
        step.fwd()
        step.bwd()
    torch.cuda.synchronize()
    graphs = _capture_step(step) if use_graph else None
    fwd_fn, bwd_fn = graphs if graphs is not None else (step.fwd, step.bwd)
    stream = torch.cuda.current_stream()
    events = []
    torch.cuda.synchronize()
    for _ in range(steps):
        ev = [StreamEvent() for _ in range(4)]
        flush_caches()
        ev[0].record(stream)
        fwd_fn()
        ev[1].record(stream)
        flush_caches()
        ev[2].record(stream)
        bwd_fn()
        ev[3].record(stream)
        events.append(ev)
    torch.cuda.synchronize()
    total = Samples([e[0].elapsed_time(e[1]) + e[2].elapsed_time(e[3]) for e in events])
    per = {k: Samples([e[a].elapsed_time(e[b]) for e in events]) for k, (a, b) in
           {"fwd": (0, 1), "bwd": (2, 3)}.items()}
    if graphs is None:
        # the backward's two launches apart: the same protocol, an event between them
        split = []
        for _ in range(steps):
            ev = [StreamEvent() for _ in range(3)]
            flush_caches()
            ev[0].record(stream)
            step.bwd_delta()
            ev[1].record(stream)
            step.bwd_main()
            ev[2].record(stream)
            split.append(ev)
        torch.cuda.synchronize()
        per["bwd_delta"] = Samples([e[0].elapsed_time(e[1]) for e in split])
        per["bwd_main"] = Samples([e[1].elapsed_time(e[2]) for e in split])
    kernel_ms = {k: v.median_ms for k, v in per.items()}
    kernel_mean_ms = {k: v.mean_ms for k, v in per.items()}
    # the same steps back to back, caches warm, wall clock
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fwd_fn()
        bwd_fn()
    torch.cuda.synchronize()
    warm = (time.perf_counter() - t0) * 1e3 / steps
    return {"step_ms": {"median": total.median_ms, "p20": total.p20_ms, "p80": total.p80_ms,
                        "mean": total.mean_ms},
            "kernel_ms": kernel_ms, "kernel_mean_ms": kernel_mean_ms, "warm_ms_per_step": warm,
            "launch": "hip_graph" if graphs is not None else "eager"}


def host_threads() -> dict:
    """Give torch's CPU ops os.cpu_count() threads (BASELINE.md's CPU plan)
    and return the counts: the threads used, the cores this process may run
    on (affinity) and the machine's total logical cores."""
    import torch
    total = os.cpu_count() or 1
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else total
    torch.set_num_threads(total)
    return {"threads": torch.get_num_threads(), "affinity_cores": affinity, "total_cores": total}


def cpu_baseline(B, H, n, bs, budget_s: float):
    """fp32 eager oracle fwd+bwd over (b, h) slices of the workload until the
    budget is spent; value in useful TFLOP/s (same FLOP convention)."""
    import torch
    from oracle.attention import bd3_attention_grads
    cores = host_threads()
    g = torch.Generator().manual_seed(0)
    q, k, v, do = (torch.randn(1, 1, 2 * n, D, generator=g).to(torch.bfloat16).float() for _ in range(4))
    bd3_attention_grads(q, k, v, do, bs)  # warmup (allocations)
    done, t0 = 0, time.perf_counter()
    while True:
        bd3_attention_grads(q, k, v, do, bs)
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s or done >= B * H:
            break
    flops = 3.5 * useful_fwd_flops(1, 1, n, bs) * done
    # forward alone (BASELINE's CPU plan times fwd and fwd+bwd)
    from oracle.attention import bd3_attention
    with torch.no_grad():
        bd3_attention(q, k, v, bs)
        f_done, f0 = 0, time.perf_counter()
        while True:
            bd3_attention(q, k, v, bs)
            f_done += 1
            f_el = time.perf_counter() - f0
            if f_el >= budget_s / 3 or f_done >= B * H:
                break
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": flops / el / 1e12,
        "unit": "TFLOP/s",
        "cores": cores["threads"],
        "host": cores,
        "kind": "port",
        "sample": (f"{done} of {B * H} (b,h) slices of the B={B} L={n} H={H} bs={bs} workload, "
                   f"fp32 eager fwd+bwd (torch autograd, {cores['threads']} threads, {cpu_model}); "
                   f"{el:.1f} s"),
        "fwd_value": useful_fwd_flops(1, 1, n, bs) * f_done / f_el / 1e12,
        "fwd_sample": f"{f_done} (b,h) slices, fp32 eager forward only; {f_el:.1f} s",
    }


def decode_cpu_baseline(budget_s: float):
    """The fp32 eager decode oracle on the host cores over (sequence, head)
    slices of configs[3] (q_len 16 over kv_len 4112) until the budget is
    spent; value in K+V GB/s (the GPU metric's byte convention)."""
    import torch
    from oracle.attention import decode_attention
    cores = host_threads()
    H, q_len, kv_len, bs = 12, 16, 4112, 16
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, H, q_len, D, generator=g).to(torch.bfloat16).float()
    k, v = (torch.randn(1, H, kv_len, D, generator=g).to(torch.bfloat16).float() for _ in range(2))
    with torch.no_grad():
        decode_attention(q, k, v, bs)
        done, t0 = 0, time.perf_counter()
        while True:
            decode_attention(q, k, v, bs)
            done += 1
            el = time.perf_counter() - t0
            if el >= budget_s or done >= 32:
                break
    nbytes = 2 * H * kv_len * D * 2 * done
    return {"value": nbytes / el / 1e9, "unit": "GB/s", "cores": cores["threads"], "host": cores, "kind": "port",
            "sample": f"{done} of 32 sequences (12 heads each) of configs[3], fp32 eager decode; {el:.2f} s"}


def decode_bench(device, reps: int):
    """32 sequences x 12 heads, 16 queries over 4096 + 16 cached keys."""
    import torch
    from kernels._native import check, lib, ptr, stream_of, strides
    from perf.harness import bench
    B, H, q_len, kv_len, bs = 32, 12, 16, 4112, 16
    q = seeded_bf16((B, H, q_len, D), 0, 1, device)[0]
    k, v = seeded_bf16((B, H, kv_len, D), 1, 2, device)
    o = torch.empty_like(q)
    kv_bytes = 2 * B * H * kv_len * D * 2
    st = strides(q, k, v, o)
    stream = stream_of(q)
    L = lib()
    rows = []

    def run(n_splits):
        nbytes = L.bd3_decode_workspace_bytes(B, H, q_len, kv_len, D, n_splits)
        ws = torch.empty(max(nbytes, 1), device=device, dtype=torch.uint8)

        def call():
            check(L.bd3_decode_splitkv(ptr(q), ptr(k), ptr(v), ptr(o), B, H, q_len, kv_len, D, bs,
                                       n_splits, st, 1.0 / 8, ptr(ws), nbytes, stream))
        return call

    # At this shape (384 batch*heads) 2 or 3 splits write fp32 partials to HBM
    # and merge them in a second launch (the reference's split_kv_kern +
    # split_kv_reduce_kern); from 4 splits on one workgroup per head takes all
    # of its splits and merges them on chip.
    for ns in (1, 2, 3, 4, 8, 16, 0):
        eff = ns if ns else -(-kv_len // 256)  # 0: the reference's SPLIT_N = 256 rule
        t = bench(run(eff), warmup=5, rep=reps, flush=True)
        merge = "none" if eff == 1 else ("partials in HBM + merge launch" if eff < 4 else "on chip, per head")
        rows.append({"n_splits": eff, "rule": "reference ceil(kv/256)" if ns == 0 else "explicit",
                     "merge": merge, "us": t.mean_ms * 1e3, "us_median": t.median_ms * 1e3,
                     "us_p20": t.p20_ms * 1e3, "us_p80": t.p80_ms * 1e3,
                     "GB_s": kv_bytes / (t.mean_ms * 1e-3) / 1e9})
    # the library's auto split (bd3_decode)
    nb_auto = L.bd3_decode_workspace_bytes(B, H, q_len, kv_len, D, 0)
    ws_auto = torch.empty(max(nb_auto, 1), device=device, dtype=torch.uint8)
    auto_splits = L.bd3_decode_auto_splits(B, H, q_len, kv_len)

    def call_auto():
        check(L.bd3_decode(ptr(q), ptr(k), ptr(v), ptr(o), B, H, q_len, kv_len, D, bs, st, 1.0 / 8,
                           ptr(ws_auto), nb_auto, stream))
    t = bench(call_auto, warmup=5, rep=reps, flush=True)
    rows.append({"n_splits": auto_splits, "rule": "auto (bd3_decode)", "us": t.mean_ms * 1e3,
                 "us_median": t.median_ms * 1e3, "us_p20": t.p20_ms * 1e3, "us_p80": t.p80_ms * 1e3,
                 "GB_s": kv_bytes / (t.mean_ms * 1e-3) / 1e9})
    best = max(rows, key=lambda r: r["GB_s"])
    return {
        "workload": "split-KV decode, 32 seq x 12 heads, q_len 16, kv_len 4112, d 64, bs 16, bf16",
        "kv_bytes": kv_bytes,
        "rows": rows,
        "roofline": {"bound": "hbm", "achieved": best["GB_s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": best["GB_s"] / PEAK_HBM_GBS, "traffic": measured_traffic("decode16_partial"),
                     "kernel": f"bd3_decode_splitkv n_splits={best['n_splits']} ({best['rule']})"},
    }


def decode_b1_bench(device, reps: int):
    """The reference's decode profiling shapes (bench/decode_ncu.py:16-19):
    batch 1, 12 heads, block 16; `cached`: a 16-token block over a 3584-token
    cache, `uncached`: the whole 3088-token sequence block-causal. Each through
    the bsdfa path (bd3_decode, automatic split count) and the split_kv path
    (the reference rule: ceil(kv_len / 256) splits, prefill falls back to
    bsdfa as the reference does, kernels/SplitKVDecodeAttention.py:140-147).
    HIP events, 1 GiB cache eviction before each call; KV-read GB/s counts the
    K and V bytes the rows can see."""
    import torch
    from kernels.BlockSparseDecodeAttention import block_sparse_decode_attention
    from kernels.SplitKVDecodeAttention import split_kv_decode_attention
    from kernels._native import lib
    from perf.harness import bench
    out = {}
    for shape, (q_len, kv_len) in (("cached", (16, 3584)), ("uncached", (3088, 3088))):
        (q,) = seeded_bf16((1, 12, q_len, D), 3, 1, device)
        k, v = seeded_bf16((1, 12, kv_len, D), 4, 2, device)
        kv_bytes = 2 * 12 * kv_len * D * 2
        for name, fn, splits in (
                ("bsdfa", block_sparse_decode_attention, lib().bd3_decode_auto_splits(1, 12, q_len, kv_len)),
                ("split_kv", split_kv_decode_attention, -(-kv_len // 256) if q_len <= 64 else "bsdfa fallback")):
            t = bench(lambda: fn(q, k, v, 16), warmup=5, rep=reps, flush=True)
            out[f"{shape}_{name}"] = {"q_len": q_len, "kv_len": kv_len, "heads": 12, "n_splits": splits,
                                      "us": t.median_ms * 1e3, "us_p20": t.p20_ms * 1e3, "us_p80": t.p80_ms * 1e3,
                                      "kv_GB_s": kv_bytes / (t.median_ms * 1e-3) / 1e9}
        del q, k, v
        torch.cuda.empty_cache()
    return out


def kvcache_bench(device, reps: int):
    """Attention inputs of one layer: head split + RoPE + KV-cache placement
    (bd3_qkv_rope) against the reference's eager path on the same GPU
    (model/modules.py:395-414: rearrange, RoPE as bf16 tensor ops, then
    torch.cat of the cache and the block for k and v).
      decode_step: configs[3]'s step, 32 sequences x 12 heads, a 16-token
        block over a 4096-token cache; ours writes q and places the block's
        k / v in the cache slot, the reference copies the whole cache.
      full_sequence: 8 x 2048 tokens x 12 heads (configs[1]'s shape) with no
        cache; HBM-bound (reads the projection, writes q, k, v once).
    `kernel_us` times the C-ABI call alone, `call_us` the Python
    attention_inputs wrapper; HIP events, 1 GiB cache flush before each rep."""
    import torch
    from kernels._native import check, lib, ptr, stream_of, strides
    from kernels.kv_cache import KVCache, attention_inputs, rope_tables
    from perf.harness import bench
    H, L_ = 12, lib()
    sin, cos = rope_tables(D, 8192, device=device)
    out = {}

    def eager(qkv, kc, vc, pos0):
        B, S, _ = qkv.shape
        q, k, v = qkv.view(B, S, 3, H, D).permute(2, 0, 3, 1, 4)
        pos = torch.arange(pos0, pos0 + S, device=device)
        s_, c_ = sin[pos].to(torch.bfloat16), cos[pos].to(torch.bfloat16)

        def rope(x):
            x1, x2 = x.chunk(2, dim=-1)
            return torch.cat([x1 * c_ - x2 * s_, x1 * s_ + x2 * c_], dim=-1)
        q, k = rope(q), rope(k)
        if kc is not None:
            k, v = torch.cat([kc, k], dim=-2), torch.cat([vc, v], dim=-2)
        return q, k, v

    for name, (B, S, L) in (("decode_step", (32, 16, 4096)), ("full_sequence", (8, 2048, 0))):
        (qkv,) = seeded_bf16((B, S, 3 * H * D), 5, 1, device)
        q = torch.empty((B, H, S, D), device=device, dtype=torch.bfloat16)
        kc = vc = None
        if L:
            kc, vc = seeded_bf16((B, H, L, D), 6, 2, device)
            cache = KVCache.empty(1, capacity=L + S)
            cache.append(0, kc, vc)
            ks, vs = cache.slot(0, q, S)
        else:
            cache = None
            ks, vs = torch.empty_like(q), torch.empty_like(q)
        xs = (ctypes.c_int64 * 2)(qkv.stride(0), qkv.stride(1))
        st = strides(q, ks, vs)
        stream = stream_of(qkv)

        def kern():
            check(L_.bd3_qkv_rope(ptr(qkv), xs, B, S, H, D, None, L, ptr(sin), ptr(cos), sin.shape[0],
                                  ptr(q), ptr(ks), ptr(vs), st, stream))

        def call():
            attention_inputs(qkv, H, sin, cos, L, cache, 0, False)

        t_k = bench(kern, warmup=3, rep=reps, flush=True)
        t_c = bench(call, warmup=3, rep=reps, flush=True)
        t_e = bench(lambda: eager(qkv, kc, vc, L), warmup=3, rep=reps, flush=True)
        nbytes = 2 * qkv.numel() * 2  # projection read once, q / k / v written once
        row = {"batch": B, "tokens": S, "heads": H, "cache_len": L,
               "kernel_us": t_k.median_ms * 1e3, "call_us": t_c.median_ms * 1e3,
               "reference_eager_us": t_e.median_ms * 1e3, "algorithmic_bytes": nbytes,
               "kernel_GB_s": nbytes / (t_k.median_ms * 1e-3) / 1e9}
        if L:
            row["reference_eager_bytes"] = nbytes + 2 * 2 * kc.numel() * 2  # + cat: read and write both caches
        out[name] = row
        del qkv, q, kc, vc, cache, ks, vs
        torch.cuda.empty_cache()
    full = out["full_sequence"]
    out["roofline"] = {"bound": "hbm", "achieved": full["kernel_GB_s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                       "frac": full["kernel_GB_s"] / PEAK_HBM_GBS, "traffic": measured_traffic("qkv_rope_kernel"),
                       "kernel": "qkv_rope_kernel (full_sequence)"}
    return out


def sampling_bench(device, reps: int):
    """One ancestral denoising step's SUBS + draw (bd3_subs_sample) against
    the reference's eager path on the same GPU (model/subs.py:11-43 with the
    reference's log_softmax, then sample/sampler.py:110-122 and :11-34 in
    float64), at configs[4]'s step (8 sequences x 32-token blocks) and
    configs[3]'s (32 x 16), vocab 50258, bf16 logits, 3/4 of the tokens
    masked. `fused_philox_us`: noise drawn in-kernel; `fused_u_us`: the
    caller's float64 uniforms read instead; `reference_eager_us` includes its
    torch.rand_like draw. HIP events, 1 GiB cache flush before each rep."""
    import torch
    from kernels.sampling import PhiloxStream, subs_sample_step
    from perf.harness import bench
    V, mask = 50258, 50257
    out = {}
    for name, (B, L) in (("config4_step", (8, 32)), ("config3_step", (32, 16))):
        g = torch.Generator(device=device).manual_seed(0)
        logits = (torch.randn(B, L, V, device=device, generator=g) * 4).to(torch.bfloat16)
        block = torch.randint(0, V - 1, (B, L), device=device, generator=g)
        block[torch.rand(B, L, device=device, generator=g) < 0.75] = mask
        u = torch.rand(B, L, V, device=device, dtype=torch.float64, generator=g)
        keep = 0.5
        gen = PhiloxStream(seed=1)

        def eager():
            bias = torch.zeros(V, device=device, dtype=logits.dtype)
            bias[mask] = -1e6
            x = logits + bias
            sh = x - x.amax(dim=-1, keepdim=True)
            lp = sh.float() - torch.log(torch.exp(sh.float()).sum(dim=-1, keepdim=True))
            carry = torch.full_like(lp, -1e6).scatter(-1, block.unsqueeze(-1), 0.0)
            lp = torch.where((block != mask).unsqueeze(-1), carry, lp)
            q = torch.exp(lp).double() * (1 - keep)
            q[..., mask] = keep
            uu = torch.rand_like(q)
            new = torch.argmax(q / (1e-10 - torch.log(uu + 1e-10)), dim=-1)
            return torch.where(block != mask, block, new)

        t_p = bench(lambda: subs_sample_step(logits, block, mask, keep, generator=gen), warmup=3, rep=reps,
                    flush=True)
        t_u = bench(lambda: subs_sample_step(logits, block, mask, keep, u=u), warmup=3, rep=reps, flush=True)
        t_e = bench(eager, warmup=3, rep=reps, flush=True)
        nbytes = logits.numel() * 2
        out[name] = {"rows": B * L, "vocab": V, "fused_philox_us": t_p.median_ms * 1e3,
                     "fused_u_us": t_u.median_ms * 1e3, "reference_eager_us": t_e.median_ms * 1e3,
                     "logits_bytes": nbytes,
                     "fused_philox_GB_s": nbytes / (t_p.median_ms * 1e-3) / 1e9}
        del logits, block, u
        torch.cuda.empty_cache()
    return out


def glue_bench(device, reps: int):
    """The DiT block's glue around attention at configs[1]'s training shape
    (8 x 2048 tokens, d_model 768; fp32 residual, bf16 adaLN vectors, bf16
    result for the next matmul) and configs[4]'s sampling step (8 x 32
    tokens, all bf16): bd3_ln_modulate and bd3_gate_residual against the
    reference's eager ops on the same GPU (model/modules.py:243-288,
    :778-788, :560-566), and the two fused (bd3_gate_residual_ln_modulate).
    HIP events, 1 GiB cache flush before each rep."""
    import torch
    from kernels.dit_glue import gate_residual, gate_residual_ln_modulate, ln_modulate
    from perf.harness import bench
    out = {}
    for name, (B, S, xd) in (("training", (8, 2048, torch.float32)), ("sampling_step", (8, 32, torch.bfloat16))):
        D = 768
        g = torch.Generator(device=device).manual_seed(0)
        x = torch.randn(B, S, D, device=device, generator=g).to(xd)
        w = torch.rand(D, device=device, generator=g) + 0.5
        sh, sc, gt = (torch.randn(B, 1, D, device=device, generator=g).to(torch.bfloat16) for _ in range(3))
        y = torch.randn(B, S, D, device=device, generator=g).to(torch.bfloat16)

        def eager_ln():
            xf = x.float()
            num = xf - xf.mean(dim=-1, keepdim=True)
            inv = torch.rsqrt(xf.var(dim=-1, keepdim=True, correction=0) + 1e-5)
            h = (w * num * inv).to(x.dtype)
            return (h * (1 + sc) + sh).to(torch.bfloat16)

        t_ln = bench(lambda: ln_modulate(x, w, sh, sc, out_dtype=torch.bfloat16), warmup=3, rep=reps, flush=True)
        t_ln_e = bench(eager_ln, warmup=3, rep=reps, flush=True)
        t_gr = bench(lambda: gate_residual(x, gt, y), warmup=3, rep=reps, flush=True)
        t_gr_e = bench(lambda: x + gt * y, warmup=3, rep=reps, flush=True)
        t_fu = bench(lambda: gate_residual_ln_modulate(x, gt, y, w, sh, sc, out_dtype=torch.bfloat16), warmup=3,
                     rep=reps, flush=True)
        xb = x.element_size()
        ln_bytes = B * S * D * (xb + 2)            # x read, bf16 result written
        gr_bytes = B * S * D * (2 * xb + 2)        # x and y read, result (x's dtype) written
        out[name] = {"batch": B, "tokens": S, "d_model": D, "x_dtype": str(xd).replace("torch.", ""),
                     "ln_modulate_us": t_ln.median_ms * 1e3, "ln_modulate_reference_eager_us": t_ln_e.median_ms * 1e3,
                     "ln_modulate_GB_s": ln_bytes / (t_ln.median_ms * 1e-3) / 1e9,
                     "gate_residual_us": t_gr.median_ms * 1e3, "gate_residual_reference_eager_us": t_gr_e.median_ms * 1e3,
                     "gate_residual_GB_s": gr_bytes / (t_gr.median_ms * 1e-3) / 1e9,
                     "gate_residual_ln_modulate_us": t_fu.median_ms * 1e3}
        del x, y
        torch.cuda.empty_cache()
    tr = out["training"]
    out["roofline"] = {"bound": "hbm", "achieved": tr["ln_modulate_GB_s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                       "frac": tr["ln_modulate_GB_s"] / PEAK_HBM_GBS, "traffic": measured_traffic("ln_modulate_kernel"),
                       "kernel": "ln_modulate_kernel (training)"}
    return out


def census(n, bs):
    """Useful and executed pairs per (b, h) of each training kernel's
    schedule (bd3_train_tile_census)."""
    from kernels._native import lib
    out = (ctypes.c_int64 * 8)()
    lib().bd3_train_tile_census(n, bs, out)
    return {"useful_pairs": out[0], "executed_pairs": {"fwd": out[1], "bwd_dq_items": out[6],
                                                        "bwd_dkdv_items": out[7]},
            "useful_fraction_of_executed": {"fwd": out[0] / out[1], "bwd_dq_items": out[0] / out[6],
                                            "bwd_dkdv_items": out[0] / out[7]}}


def train_record(step: "TrainStep", t: dict) -> dict:
    """Throughput figures of one timed training configuration.

    useful: 3.5 x the useful forward FLOPs 4*d*B*H*(n^2 + n*bs) per step
    (backward credited 2.5x forward, bench/attention_bench.py:89,99, counted on
    unmasked pairs only). reference_convention: the reference microbench's
    own figures, dense FLOPs 4*B*H*L^2*d with L = 2n, fwd_tflops =
    fwd_flops / fwd time, bwd_tflops = 2.5 fwd_flops / bwd time
    (bench/attention_bench.py:89,98-99). kernel_formed_tflops: the products
    each kernel forms (forward S, PV; the backward's main launch S, dP, dQ for
    its dQ items and S, dP, dV, dK for its dK/dV items: recomputation
    included) per second."""
    B, H, n, bs = step.B, step.H, step.n, step.bs
    fwd = useful_fwd_flops(B, H, n, bs)
    ms = t["step_ms"]["median"]
    rec = {"ms_per_step": ms, "step_ms": t["step_ms"], "warm_ms_per_step": t["warm_ms_per_step"],
           "launch": t["launch"], "kernel_ms": t["kernel_ms"], "kernel_mean_ms": t["kernel_mean_ms"],
           "useful_tflops": 3.5 * fwd / (ms * 1e-3) / 1e12,
           "frac_of_peak": 3.5 * fwd / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
           "census": census(n, bs)}
    km = t["kernel_ms"]
    if km:
        dense = 4 * B * H * (2 * n) ** 2 * D
        bwd_ms = km["bwd"]
        rec["useful_fwd_tflops"] = fwd / (km["fwd"] * 1e-3) / 1e12
        rec["useful_bwd_tflops"] = 2.5 * fwd / (bwd_ms * 1e-3) / 1e12
        rec["reference_convention"] = {"fwd_ms": km["fwd"], "bwd_ms": bwd_ms, "dense_fwd_flops": dense,
                                       "fwd_tflops": dense / (km["fwd"] * 1e-3) / 1e12,
                                       "bwd_tflops": 2.5 * dense / (bwd_ms * 1e-3) / 1e12}
        formed = {"fwd": 1.0, "bwd_main": 3.5}
        rec["kernel_formed_tflops"] = {k: formed[k] * fwd / (km[k] * 1e-3) / 1e12 for k in formed if k in km}
    return rec


def sweep_bench(device, steps: int, use_graph: bool = False):
    """B=4, L=2048, H=16, block sizes {4, 16, 64, 256}."""
    import torch
    out = []
    for bs in (4, 16, 64, 256):
        st = TrainStep(4, 16, 2048, bs, device)
        t = time_train(st, steps, 2, use_graph, ramp_s=0.3)
        out.append({"block_size": bs, **train_record(st, t)})
        del st
        torch.cuda.empty_cache()
    return out


def long_bench(device, steps: int):
    """The reference microbench's sequence ladder (bench/attention_bench.py:
    15-20, :86): 16384 tokens per batch, B = 16384 / 2n, 12 heads, n in
    {1024, 2048, 4096, 8192} at block 16 and n = 4096 at blocks {4, 64, 256}."""
    import torch
    out = []
    for n, bs in [(1024, 16), (2048, 16), (4096, 16), (8192, 16), (4096, 4), (4096, 64), (4096, 256)]:
        B = max(1, 16384 // (2 * n))
        st = TrainStep(B, 12, n, bs, device)
        t = time_train(st, steps, 2, False, ramp_s=0.3)
        out.append({"n": n, "attn_seq": 2 * n, "batch": B, "block_size": bs, **train_record(st, t)})
        del st
        torch.cuda.empty_cache()
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--long", action="store_true", help="also time the reference microbench's long-sequence ladder")
    ap.add_argument("--no-kvcache", action="store_true")
    ap.add_argument("--no-sampling", action="store_true")
    ap.add_argument("--no-glue", action="store_true")
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--graph", action="store_true", help="replay the step from a captured HIP graph instead of launching it")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures the attention kernels on ONE GPU: the path has no "
              "cross-GPU exchange to measure (each (batch, head) is independent); "
              "run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    from kernels._native import lib
    metric = json.loads((REPO / "BASELINE.json").read_text())["metric"]
    device = torch.device("cuda:0")
    log(f"device: {torch.cuda.get_device_name(device)}")

    B, H, n, bs = 8, 12, 1024, 16
    step = TrainStep(B, H, n, bs, device)
    t = time_train(step, args.steps, args.warmup, use_graph=args.graph)
    rec = train_record(step, t)
    ms, per = rec["ms_per_step"], t["kernel_ms"]
    tflops = rec["useful_tflops"]
    log(f"config1 fwd+bwd ({t['launch']}, caches evicted before fwd and before bwd): {ms * 1e3:.1f} us/step median "
        f"(p20 {t['step_ms']['p20'] * 1e3:.1f}, p80 {t['step_ms']['p80'] * 1e3:.1f}; back to back warm "
        f"{t['warm_ms_per_step'] * 1e3:.1f}) -> {tflops:.1f} useful TFLOP/s")
    if "bwd_main" in per:
        log(f"  fwd {per['fwd'] * 1e3:.1f} us, bwd Delta pass {per['bwd_delta'] * 1e3:.1f} us, "
            f"bwd main launch {per['bwd_main'] * 1e3:.1f} us")

    # Dominant kernel's roofline: its algorithmic (useful) FLOPs per launch,
    # the FA2 credit of the products it owns (forward 1x the useful forward
    # FLOPs; the backward's main launch 2.5x: all of the backward's products),
    # over its average (mean) launch duration inside the timed steps.
    fwd_flops = useful_fwd_flops(B, H, n, bs)
    credit = {"fwd": 1.0, "bwd_main": 2.5}
    names = {"fwd": "attn_fwd_dma_kernel", "bwd_main": "attn_bwd_kernel"}
    per = {k: v for k, v in per.items() if k in credit}
    dom = max(per, key=per.get) if per else "bwd_main"
    dom_flops = credit[dom] * fwd_flops
    dom_mean = t["kernel_mean_ms"].get(dom)
    achieved = dom_flops / (dom_mean * 1e-3) / 1e12 if dom_mean else None

    result = {
        "metric": metric,
        "value": tflops,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: q, k, v, dO ~ N(0,1) from seed 0, bf16, resident in HBM (caches evicted before the forward and before the backward)",
        "config": {"workload": "BD3-LM training attention fwd+bwd (configs[1])", "batch": B,
                   "seq_len": n, "attn_seq": 2 * n, "heads": H, "head_dim": D, "block_size": bs},
        **{k: v for k, v in rec.items() if k not in ("ms_per_step",)},
        "kernel_useful_tflops": ({k: credit[k] * fwd_flops / (per[k] * 1e-3) / 1e12 for k in per} if per else None),
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS if achieved else None,
                     "traffic": measured_traffic(names[dom]),
                     "kernel": names[dom], "algorithmic_flops_per_launch": dom_flops,
                     "mean_launch_us": dom_mean * 1e3 if dom_mean else None,
                     "credit": f"{credit[dom]} x useful forward FLOPs (FA2 convention: backward = 2.5x forward, "
                               "all of it owned by the backward's main launch; the Delta pass owns none)"},
    }
    del step
    torch.cuda.empty_cache()

    # The clock the matrix cores hold under load (the 2.5 PFLOP/s peak above
    # assumes 2.4 GHz): measured right after the timed steps, for context.
    from perf.harness import shader_clock_ghz
    sclk = shader_clock_ghz(lib(), device)
    result["sclk_under_mfma_load"] = sclk
    if achieved:
        result["roofline"]["frac_at_measured_sclk"] = achieved / sclk["bf16_peak_tflops"]
    log(f"shader clock under MFMA load: {sclk['median']:.3f} GHz (min {sclk['min']:.3f}, max {sclk['max']:.3f}) "
        f"-> bf16 dense peak {sclk['bf16_peak_tflops']:.0f} TFLOP/s")

    if not args.no_decode:
        result["decode"] = decode_bench(device, reps=30)
        for r in result["decode"]["rows"]:
            log(f"decode n_splits={r['n_splits']:3d} ({r['rule']}, merge {r.get('merge', 'none')}): "
                f"{r['us']:.1f} us, {r['GB_s']:.0f} GB/s")
    if not args.no_decode:
        result["decode_batch1"] = decode_b1_bench(device, reps=30)
        for k_, r in result["decode_batch1"].items():
            log(f"decode batch-1 {k_}: {r['us']:.1f} us ({r['kv_GB_s']:.0f} GB/s, splits {r['n_splits']})")
    if not args.no_kvcache:
        result["kv_cache"] = kvcache_bench(device, reps=20)
        for k_, r in result["kv_cache"].items():
            if k_ != "roofline":
                log(f"kv_cache {k_}: kernel {r['kernel_us']:.1f} us ({r['kernel_GB_s']:.0f} GB/s), "
                    f"call {r['call_us']:.1f} us, reference eager {r['reference_eager_us']:.1f} us")
    if not args.no_sampling:
        result["sampling"] = sampling_bench(device, reps=20)
        for k_, r in result["sampling"].items():
            log(f"sampling {k_}: fused {r['fused_philox_us']:.1f} us (philox) / {r['fused_u_us']:.1f} us (given u), "
                f"reference eager {r['reference_eager_us']:.1f} us")
    if not args.no_glue:
        result["dit_glue"] = glue_bench(device, reps=20)
        for k_, r in result["dit_glue"].items():
            if k_ != "roofline":
                log(f"dit_glue {k_}: ln_modulate {r['ln_modulate_us']:.1f} us ({r['ln_modulate_GB_s']:.0f} GB/s, "
                    f"eager {r['ln_modulate_reference_eager_us']:.1f} us), gate_residual {r['gate_residual_us']:.1f} us "
                    f"({r['gate_residual_GB_s']:.0f} GB/s, eager {r['gate_residual_reference_eager_us']:.1f} us), "
                    f"fused {r['gate_residual_ln_modulate_us']:.1f} us")
    if not args.no_e2e:
        from perf.e2e_sampling import run as e2e_run
        result["e2e"] = e2e_run(blocks=64, eager_blocks=2, check_steps=4)
        worst = max(d["max_abs"] for d in result["e2e"]["logit_check"])
        log(f"e2e configs[4]: {result['e2e']['tokens_per_s']:.0f} tokens/s "
            f"(reference eager path {result['e2e']['reference_eager_tokens_per_s']:.0f} tokens/s), "
            f"logit max-abs vs eager {worst:.4g}")
        torch.cuda.empty_cache()
    if not args.no_sweep:
        result["sweep"] = sweep_bench(device, steps=10, use_graph=args.graph)
        for r in result["sweep"]:
            log(f"sweep bs={r['block_size']:3d}: {r['ms_per_step'] * 1e3:.1f} us, {r['useful_tflops']:.1f} TFLOP/s")
    if args.long:
        result["long_sequences"] = long_bench(device, steps=10)
        for r in result["long_sequences"]:
            log(f"long n={r['n']:5d} B={r['batch']} bs={r['block_size']:3d}: {r['ms_per_step'] * 1e3:.1f} us, "
                f"{r['useful_tflops']:.1f} useful TFLOP/s; reference convention fwd "
                f"{r['reference_convention']['fwd_tflops']:.0f} / bwd {r['reference_convention']['bwd_tflops']:.0f} TFLOP/s")
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(B, H, n, bs, args.cpu_budget)
        if "decode" in result:
            result["decode"]["cpu_baseline"] = decode_cpu_baseline(args.cpu_budget / 3)
            log(f"decode cpu baseline: {result['decode']['cpu_baseline']['value']:.1f} GB/s")
        log(f"cpu baseline: {result['cpu_baseline']['value'] * 1e3:.2f} GFLOP/s "
            f"({result['cpu_baseline']['sample']})")
    else:
        result["cpu_baseline"] = None
    log_sections(result)
    print(json.dumps(result), flush=True)
    return 0


def log_sections(result: dict) -> None:
    """One JSONL record per bench section in RESULTS_DIR (perf.harness.log_result,
    the reference's bench/harness.py:75-91 record: config, timing, environment
    and the section's figures)."""
    from perf.harness import RESULTS_DIR, log_result
    train = {k: v for k, v in result.items()
             if k not in ("config", "decode", "decode_batch1", "kv_cache", "sampling", "dit_glue", "e2e", "sweep",
                          "long_sequences")}
    log_result("attention_train", result["config"], timing=result.get("step_ms"), **train)
    for key in ("decode", "decode_batch1", "kv_cache", "sampling", "dit_glue", "e2e", "sweep", "long_sequences"):
        if key in result:
            log_result(key, {"workload": key}, figures=result[key])
    log(f"results appended to {RESULTS_DIR}/*.jsonl")


if __name__ == "__main__":
    sys.exit(main())
