"""Short, fixed workload for rocprofv3 counter runs (--pmc).

    rocprofv3 --pmc FETCH_SIZE -- python3 diffusion-llm_amd/perf/pmc_workload.py

Dispatches, in order and each `--reps` times:
  1. a plain device copy of --copy-mib MiB (torch copy_) - the calibration
     kernel: its FETCH_SIZE / WRITE_SIZE per dispatch against its known
     byte count gives the factor that turns the counters into bytes;
  2. the training forward and the backward (its Delta pass and its main
     launch of every dQ and dK/dV item), by default at BASELINE
     configs[1] (B=8, L=1024, H=12, d=64, block 16, bf16; --batch, --heads,
     --seq-len and --block-size change the shape);
  3. the split-KV decode at configs[3] (32 x 12 heads, q_len 16,
     kv_len 4112) with the library's automatic split count;
  4. the layer's attention inputs (bd3_qkv_rope: head split + RoPE) over a
     full 8 x 2048-token sequence, 12 heads;
  5. LayerNorm + adaLN modulate (bd3_ln_modulate) over 8 x 2048 tokens of
     d_model 768 (fp32 residual, bf16 vectors, bf16 result).
With --decode-b1 only (no calibration copy, training or other kernels): the
reference's decode profiling shapes (bench/decode_ncu.py:16-19), batch 1,
12 heads, block 16 - a 16-token block over a 3584-token cache and the whole
3088-token sequence block-causal - each through bd3_decode (automatic split
count) and the split_kv path (the reference rule ceil(kv_len / 256) for the
cached shape; prefill falls back to the block-sparse path as the reference
does, kernels/SplitKVDecodeAttention.py:140-147).
No timing is done here; the profiler records per-dispatch counters (or, under
--kernel-trace --stats, durations).
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

_HERE = Path(__file__).resolve()
for _p in (str(_HERE.parents[2]), str(_HERE.parents[1])):
    if _p not in sys.path:
        sys.path.insert(0, _p)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--heads", type=int, default=12)
    ap.add_argument("--seq-len", type=int, default=1024)
    ap.add_argument("--block-size", type=int, default=16)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--decode-b1", action="store_true", help="only the batch-1 decode profiling shapes")
    args = ap.parse_args(argv)

    import torch
    from bench import TrainStep, seeded_bf16
    from kernels._native import check, lib, ptr, stream_of, strides

    dev = torch.device("cuda:0")
    if args.decode_b1:
        return decode_b1(args.reps, dev)
    n_el = args.copy_mib * (1 << 20) // 4
    src = torch.ones(n_el, device=dev, dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(args.reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copy calibration: {args.copy_mib} MiB read + {args.copy_mib} MiB written per dispatch", flush=True)

    step = TrainStep(args.batch, args.heads, args.seq_len, args.block_size, dev)
    for _ in range(args.reps):
        step.fwd()
        step.bwd()
    torch.cuda.synchronize()
    print("training kernels done", flush=True)
    del step

    if args.no_decode:
        return 0
    B, H, q_len, kv_len, bs, D = 32, 12, 16, 4112, 16, 64
    q = seeded_bf16((B, H, q_len, D), 0, 1, dev)[0]
    k, v = seeded_bf16((B, H, kv_len, D), 1, 2, dev)
    o = torch.empty_like(q)
    L = lib()
    nbytes = L.bd3_decode_workspace_bytes(B, H, q_len, kv_len, D, 0)
    ws = torch.empty(max(nbytes, 1), device=dev, dtype=torch.uint8)
    st = strides(q, k, v, o)
    for _ in range(args.reps):
        check(L.bd3_decode(ptr(q), ptr(k), ptr(v), ptr(o), B, H, q_len, kv_len, D, bs, st, 1.0 / 8,
                           ptr(ws), nbytes, stream_of(q)))
    torch.cuda.synchronize()
    print(f"decode done (K+V bytes per dispatch {2 * B * H * kv_len * D * 2})", flush=True)
    del q, k, v, o, ws

    import ctypes
    from kernels.kv_cache import rope_tables
    B, S, H = 8, 2048, 12
    (qkv,) = seeded_bf16((B, S, 3 * H * D), 5, 1, dev)
    sin, cos = rope_tables(D, S, device=dev)
    qo, ko, vo = (torch.empty((B, H, S, D), device=dev, dtype=torch.bfloat16) for _ in range(3))
    xs = (ctypes.c_int64 * 2)(qkv.stride(0), qkv.stride(1))
    st = strides(qo, ko, vo)
    for _ in range(args.reps):
        check(L.bd3_qkv_rope(ptr(qkv), xs, B, S, H, D, None, 0, ptr(sin), ptr(cos), S, ptr(qo), ptr(ko),
                             ptr(vo), st, stream_of(qkv)))
    torch.cuda.synchronize()
    print(f"qkv_rope done (projection bytes read per dispatch {qkv.numel() * 2})", flush=True)
    del qkv, qo, ko, vo

    from kernels.dit_glue import ln_modulate
    x = torch.randn(8, 2048, 768, device=dev)
    w = torch.ones(768, device=dev)
    sh = torch.zeros(8, 1, 768, device=dev, dtype=torch.bfloat16)
    for _ in range(args.reps):
        ln_modulate(x, w, sh, sh, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    print(f"ln_modulate done (x bytes read per dispatch {x.numel() * 4})", flush=True)
    return 0


def decode_b1(reps: int, dev) -> int:
    import torch
    from bench import seeded_bf16
    from kernels.BlockSparseDecodeAttention import block_sparse_decode_attention
    from kernels.SplitKVDecodeAttention import split_kv_decode_attention
    D = 64
    for shape, (q_len, kv_len) in (("cached", (16, 3584)), ("uncached", (3088, 3088))):
        (q,) = seeded_bf16((1, 12, q_len, D), 3, 1, dev)
        k, v = seeded_bf16((1, 12, kv_len, D), 4, 2, dev)
        for name, fn in (("bsdfa", block_sparse_decode_attention), ("split_kv", split_kv_decode_attention)):
            for _ in range(reps):
                fn(q, k, v, 16)
            torch.cuda.synchronize()
            print(f"decode batch 1 {shape} ({q_len} over {kv_len}) via {name}: {reps} calls", flush=True)
        del q, k, v
    return 0


if __name__ == "__main__":
    sys.exit(main())
