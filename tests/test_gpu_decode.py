"""Decode attention (families D1, D2) on the GPU against the fp32 oracle.

Bar: bf16 outputs within 2e-2 max-abs of the eager oracle (decode mask =
the block-causal slice of the training mask), split-count invariance.
"""
import pytest
import torch

from _gpu_util import max_abs, splitkv_capi
from kernels.BlockSparseDecodeAttention import block_sparse_decode_attention
from kernels.SplitKVDecodeAttention import split_kv_decode_attention
from kernels._native import check, lib, ptr, stream_of, strides
from oracle.attention import bf16_round, decode_attention, seeded_normal

OUT_TOL = 2e-2


def decode_inputs(B, H, q_len, kv_len, seed):
    g = torch.Generator().manual_seed(seed)
    q = bf16_round(torch.randn(B, H, q_len, 64, generator=g))
    k = bf16_round(torch.randn(B, H, kv_len, 64, generator=g))
    v = bf16_round(torch.randn(B, H, kv_len, 64, generator=g))
    return q, k, v


CASES = [(2, 3, 16, 300, 16), (1, 2, 16, 16, 16), (2, 2, 32, 2048, 32), (1, 2, 1, 37, 4),
         (1, 1, 200, 200, 16), (1, 2, 100, 300, 7), (2, 2, 64, 4112, 16), (1, 1, 130, 515, 64)]


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,q_len,kv_len,bs", CASES)
def test_decode_matches_oracle(cuda, B, H, q_len, kv_len, bs):
    q, k, v = decode_inputs(B, H, q_len, kv_len, seed=q_len + kv_len)
    o = block_sparse_decode_attention(*(t.to(cuda, torch.bfloat16) for t in (q, k, v)), bs)
    ref = decode_attention(q, k, v, bs)
    torch.cuda.synchronize()
    assert max_abs(o, ref) <= OUT_TOL


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,q_len,kv_len,bs", CASES)
@pytest.mark.parametrize("n_splits", [1, 2, 5, 16])
def test_splitkv_matches_oracle(cuda, B, H, q_len, kv_len, bs, n_splits):
    if n_splits > kv_len:
        pytest.skip("more splits than keys")
    q, k, v = decode_inputs(B, H, q_len, kv_len, seed=7 * q_len + kv_len)
    o = splitkv_capi(*(t.to(cuda, torch.bfloat16) for t in (q, k, v)), bs, n_splits)
    ref = decode_attention(q, k, v, bs)
    torch.cuda.synchronize()
    assert max_abs(o, ref) <= OUT_TOL


# Shapes where one workgroup takes several consecutive splits (batch * heads * n_splits > 512 and
# at least 4 splits per workgroup): ragged key counts, short or empty last splits, q_len 1..16,
# block sizes off the 16-key strips.
GROUPED = [(4, 12, 16, 1000, 16, 33), (8, 12, 7, 3001, 5, 20), (2, 16, 16, 4112, 16, 64),
           (16, 12, 1, 777, 16, 12), (8, 8, 16, 2048, 64, 40), (3, 12, 11, 1234, 3, 30)]


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,q_len,kv_len,bs,n_splits", GROUPED)
def test_grouped_splits_match_oracle(cuda, record_error, B, H, q_len, kv_len, bs, n_splits):
    """decode16_partial with several splits per workgroup (each wave's share of
    a split merged on chip, heads starting at rotated splits) against the
    oracle and against one split."""
    q, k, v = decode_inputs(B, H, q_len, kv_len, seed=B * 1000 + kv_len + n_splits)
    qd, kd, vd = (t.to(cuda, torch.bfloat16) for t in (q, k, v))
    o = splitkv_capi(qd, kd, vd, bs, n_splits)
    o1 = splitkv_capi(qd, kd, vd, bs, 1)
    ref = decode_attention(q, k, v, bs)
    torch.cuda.synchronize()
    err = max_abs(o, ref)
    record_error("decode O max-abs", err, OUT_TOL)
    assert err <= OUT_TOL
    assert max_abs(o, o1) <= 1e-2


@pytest.mark.gpu
def test_config3_split_invariance(cuda):
    """32 sequences x 12 heads, 16 queries over a
    4096 + 16 cache; splits {1, 4, 8, 16} and the reference default rule
    all match the oracle and each other."""
    B, H, q_len, kv_len, bs = 32, 12, 16, 4112, 16
    q, k, v = decode_inputs(B, H, q_len, kv_len, seed=0)
    qd, kd, vd = (t.to(cuda, torch.bfloat16) for t in (q, k, v))
    ref = decode_attention(q, k, v, bs)
    outs = [splitkv_capi(qd, kd, vd, bs, s) for s in (1, 4, 8, 16)]
    outs.append(split_kv_decode_attention(qd, kd, vd, bs))
    outs.append(block_sparse_decode_attention(qd, kd, vd, bs))
    torch.cuda.synchronize()
    for o in outs:
        assert max_abs(o, ref) <= OUT_TOL
    for o in outs[1:]:
        assert max_abs(o, outs[0]) <= 1e-2


# q_len > 64 runs the prefill kernel: 128-row query tiles, splits of whole
# 64-key tiles, row tiles whose keys fit the first split written directly and
# the others merged from partials; empty trailing splits; ragged last key
# and row tiles; per-element masks (bs or kv_len not multiples of 16).
PREFILL = [(1, 2, 1000, 1000, 16), (2, 3, 333, 2000, 5), (1, 2, 129, 4000, 32), (1, 1, 65, 65, 1),
           (1, 12, 3088, 3088, 16), (2, 2, 512, 1030, 16)]


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,q_len,kv_len,bs", PREFILL)
def test_prefill_splits_match_oracle(cuda, record_error, B, H, q_len, kv_len, bs):
    q, k, v = decode_inputs(B, H, q_len, kv_len, seed=3 * q_len + kv_len)
    ref = decode_attention(q, k, v, bs)
    dq, dk, dv = (t.to(cuda, torch.bfloat16) for t in (q, k, v))
    outs = {}
    for ns in (1, 2, 3, 7, 40):
        if ns > kv_len:
            continue
        print(f"prefill B={B} H={H} q_len={q_len} kv_len={kv_len} bs={bs} splits={ns}", flush=True)
        outs[ns] = splitkv_capi(dq, dk, dv, bs, ns)
    auto = block_sparse_decode_attention(dq, dk, dv, bs)
    torch.cuda.synchronize()
    for ns, o in outs.items():
        record_error(f"prefill O max-abs ({ns} splits)", max_abs(o, ref), OUT_TOL)
        # a split changes each P's bf16 rounding (its running maximum
        # differs) and the fp32 merge, nothing else
        assert max_abs(o, outs[1]) <= 1e-2, f"{ns} splits vs one"
    record_error("prefill O max-abs (auto splits)", max_abs(auto, ref), OUT_TOL)


def _random_prefill_shapes(count: int, seed: int):
    """(B, H, q_len, kv_len, bs, n_splits) drawn from a fixed generator:
    q_len 65-700 (the prefill kernel), a cached prefix of 0-1500 keys, block
    sizes 1-300, split counts 1-24 (many of them past the last key tile)."""
    import random
    r = random.Random(seed)
    out = []
    for _ in range(count):
        q_len = r.randint(65, 700)
        kv_len = q_len + r.choice([0, 0, r.randint(1, 1500)])
        out.append((r.randint(1, 2), r.randint(1, 3), q_len, kv_len, r.choice([1, 3, 7, 16, 32, 48, 64, 100, 300]),
                    r.randint(1, 24)))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,q_len,kv_len,bs,n_splits", _random_prefill_shapes(16, seed=2026))
def test_prefill_random_shapes(cuda, record_error, B, H, q_len, kv_len, bs, n_splits):
    print(f"prefill random B={B} H={H} q_len={q_len} kv_len={kv_len} bs={bs} splits={n_splits}", flush=True)
    q, k, v = decode_inputs(B, H, q_len, kv_len, seed=q_len * 7 + kv_len)
    o = splitkv_capi(*(t.to(cuda, torch.bfloat16) for t in (q, k, v)), bs, n_splits)
    ref = decode_attention(q, k, v, bs)
    torch.cuda.synchronize()
    record_error("prefill O max-abs (random shapes)", max_abs(o, ref), OUT_TOL)


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
@pytest.mark.parametrize("q_len", [16, 300])
def test_decode_strided_cache_view(cuda, q_len, layout):
    """K/V read in place from a larger preallocated cache equal the
    contiguous result, for the decode kernel (q_len 16) and the prefill
    kernel (q_len 300, tile loads): a (B, H, L_max, d) buffer (outer strides)
    or a (B, L_max, H, d) one (sequence stride H * d)."""
    B, H, kv_len, L_max, bs = 2, 3, 500, 1024, 16
    shape = (B, H, L_max, 64) if layout == "bhsd" else (B, L_max, H, 64)
    kc = torch.randn(shape, device=cuda, dtype=torch.bfloat16)
    vc = torch.randn(shape, device=cuda, dtype=torch.bfloat16)
    if layout == "bshd":
        kc, vc = kc.transpose(1, 2), vc.transpose(1, 2)
    q = torch.randn(B, H, q_len, 64, device=cuda, dtype=torch.bfloat16)
    o1 = block_sparse_decode_attention(q, kc[:, :, :kv_len], vc[:, :, :kv_len], bs)
    o2 = block_sparse_decode_attention(q, kc[:, :, :kv_len].contiguous(),
                                       vc[:, :, :kv_len].contiguous(), bs)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


# The reference's decode profiling shapes (bench/decode_ncu.py:16-19): batch
# 1, 12 heads, block 16 -- a 16-token block over a 3584-token cache, and the
# whole 3088-token sequence block-causal (prefill / uncached step).
NCU_SHAPES = {"cached": (16, 3584), "uncached": (3088, 3088)}


@pytest.mark.gpu
@pytest.mark.parametrize("shape", sorted(NCU_SHAPES))
@pytest.mark.parametrize("backend", ["bsdfa", "split_kv"])
def test_batch1_profiling_shapes(cuda, record_error, shape, backend):
    q_len, kv_len = NCU_SHAPES[shape]
    print(f"decode batch-1 {shape} q_len={q_len} kv_len={kv_len} via {backend}", flush=True)
    q, k, v = decode_inputs(1, 12, q_len, kv_len, seed=kv_len)
    fn = block_sparse_decode_attention if backend == "bsdfa" else split_kv_decode_attention
    o = fn(*(t.to(cuda, torch.bfloat16) for t in (q, k, v)), 16)
    ref = decode_attention(q, k, v, 16)
    torch.cuda.synchronize()
    record_error("decode O max-abs", max_abs(o, ref), OUT_TOL)


@pytest.mark.gpu
def test_cached_step_every_split_count(cuda, record_error):
    """The reference's batch-1 cached shape at every split count 1-32 (one
    partial per split, merged by decode_combine: 7-14 splits of 256-512 keys,
    ragged last splits, 17-32 splits through the 32-split merge) against the
    oracle; then 512 and 513 heads at two splits (q_len 9, block 7)."""
    q, k, v = decode_inputs(1, 12, 16, 3584, seed=11)
    ref = decode_attention(q, k, v, 16)
    qd, kd, vd = (t.to(cuda, torch.bfloat16) for t in (q, k, v))
    for ns in range(1, 33):
        print(f"decode batch 1 x 12 heads, 3584 keys, {ns} splits", flush=True)
        o = splitkv_capi(qd, kd, vd, 16, ns)
        torch.cuda.synchronize()
        record_error(f"decode O max-abs ({ns} splits)", max_abs(o, ref), OUT_TOL)
    for B, H in ((32, 16), (27, 19)):
        print(f"decode B={B} H={H} q_len 9 kv_len 300 2 splits", flush=True)
        q, k, v = decode_inputs(B, H, 9, 300, seed=B + H)
        o = splitkv_capi(*(t.to(cuda, torch.bfloat16) for t in (q, k, v)), 7, 2)
        torch.cuda.synchronize()
        record_error(f"decode O max-abs ({B * H} heads)", max_abs(o, decode_attention(q, k, v, 7)), OUT_TOL)


@pytest.mark.gpu
def test_cached_step_repeated_calls_on_two_streams(cuda):
    """600 split-KV calls, three shapes alternating over two streams, 50 calls
    in flight between synchronizations: every output equals its shape's first
    one bit for bit (the split merge is deterministic and each call's partials
    live in its own workspace)."""
    shapes = [(1, 12, 16, 3584, 16, 16), (2, 3, 16, 300, 16, 5), (4, 12, 1, 1000, 4, 7)]
    inputs, first = [], []
    for i, (B, H, q_len, kv_len, bs, ns) in enumerate(shapes):
        t = tuple(x.to(cuda, torch.bfloat16) for x in decode_inputs(B, H, q_len, kv_len, seed=90 + i))
        inputs.append(t)
        first.append(splitkv_capi(*t, bs, ns))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for batch in range(12):
        print(f"repeated split-KV calls {50 * batch}..{50 * batch + 49}", flush=True)
        outs = []
        for i in range(50):
            j = (50 * batch + i) % 3
            with torch.cuda.stream(streams[i % 2]):
                outs.append((j, splitkv_capi(*inputs[j], shapes[j][4], shapes[j][5])))
        torch.cuda.synchronize()
        for j, o in outs:
            assert torch.equal(o, first[j]), f"shape {shapes[j]} differs in call batch {batch}"


@pytest.mark.gpu
@pytest.mark.parametrize("q_len,kv_len,n_splits", [(1, 300, 1), (16, 700, 1), (16, 700, 3), (32, 1000, 2),
                                                   (300, 1100, 1), (300, 1100, 3)])
def test_decode_scale_argument(cuda, q_len, kv_len, n_splits):
    """`scale` is applied, not assumed, on every decode path (q_len 1-16,
    17-64, the prefill kernel above 64; one split and merged splits):
    doubling q and halving scale leaves the logits, hence O, bit-identical."""
    B, H, bs = 2, 3, 16
    q, k, v = (t.to(cuda, torch.bfloat16) for t in decode_inputs(B, H, q_len, kv_len, seed=q_len + kv_len))
    outs = []
    for qq, scale in ((q, 0.125), (q * 2, 0.0625)):
        o = torch.empty_like(qq)
        nbytes = lib().bd3_decode_workspace_bytes(B, H, q_len, kv_len, 64, n_splits)
        ws = torch.empty(max(nbytes, 1), device=cuda, dtype=torch.uint8)
        check(lib().bd3_decode_splitkv(ptr(qq), ptr(k), ptr(v), ptr(o), B, H, q_len, kv_len, 64, bs, n_splits,
                                       strides(qq, k, v, o), scale, ptr(ws), nbytes, stream_of(qq)))
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


@pytest.mark.gpu
@pytest.mark.parametrize("q_len,kv_len,n_splits", [(16, 700, 1), (16, 700, 3), (32, 1000, 2), (300, 1100, 1),
                                                   (300, 1100, 3)])
def test_decode_large_logits(cuda, record_error, q_len, kv_len, n_splits):
    """Scores with a standard deviation near 10 on every decode path: exact
    fp32 scores scaled in fp32, within the output bar."""
    B, H, bs = 1, 3, 16
    q, k, v = decode_inputs(B, H, q_len, kv_len, seed=q_len * 7 + n_splits)
    q = bf16_round(q * 10)
    o = splitkv_capi(*(t.to(cuda, torch.bfloat16) for t in (q, k, v)), bs, n_splits)
    ref = decode_attention(q, k, v, bs)
    torch.cuda.synchronize()
    record_error("O max-abs", max_abs(o, ref), OUT_TOL)
