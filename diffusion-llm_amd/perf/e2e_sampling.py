"""end-to-end BD3-LM block sampling with this library's kernels.

    python diffusion-llm_amd/perf/e2e_sampling.py [--blocks 64] [--check-steps 4]

A minimal restatement of the reference's inference model and sampler, used
only to measure the attention path in place (it is a benchmark workload,
not a model library): the DiT backbone (model/modules.py: Embedding, the
TimestepEmbedder, DiTBlock with adaLN, LayerNorm, RoPE attention and the GELU
MLP, FinalLayer) at 12 layers x 768 wide x 12 heads, d_ff 3072, d_cond 128,
vocab 50258 with [MASK] = 50257, and sample_bd3lm (sample/sampler.py:37-158)
with the KV cache: 8 sequences of 2048 tokens in blocks of 32, 32 denoising
steps per block plus one commit pass. Weights follow the reference's
initialisers from a seed, with two documented deviations: the adaLN
projections and lm_head are drawn like the other matmul weights instead of
zero (zero makes every block the identity and every logit 0, so a logit
comparison would be vacuous), and 2-D weights are stored in bf16 (the
reference's bf16_weights rung, inference/generate.py:28-36).

Two backbones share the weights and every non-attention op (torch matmuls,
embedding, GELU):
  * "eager": the reference's eager path - RoPE as bf16 tensor ops, cache
    growth by torch.cat, attention as fp32-logit softmax with P cast to bf16
    (model/modules.py:728-771), LayerNorm / modulate / residual as torch ops,
    SUBS + float64 Gumbel-max sampling as torch ops;
  * "bd3": this library - attention_inputs (fused QKV split + RoPE into a
    preallocated KVCache), torch.ops.bd3.decode over the cache views,
    ln_modulate / gate_residual, subs_sample_step (Philox noise).
The run reports tokens/s of the bd3 sampler over the whole generation (with
each block's backbone captured once as a HIP graph and replayed per step,
and with plain launches), the eager sampler's tokens/s over the first
blocks, and the logits' max-abs difference between the two backbones at
sampled denoising steps (same tokens, same committed prefix).
"""
from __future__ import annotations

import argparse
import json
import math
import sys
import time
from dataclasses import dataclass
from pathlib import Path

_HERE = Path(__file__).resolve()
for _p in (str(_HERE.parents[2]), str(_HERE.parents[1])):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch
import torch.nn.functional as F

BF = torch.bfloat16


@dataclass
class Cfg:
    vocab: int = 50258
    mask: int = 50257
    max_seq: int = 2048
    d: int = 768
    heads: int = 12
    layers: int = 12
    d_ff: int = 3072
    d_cond: int = 128
    freq_dim: int = 256
    bs: int = 32
    eps: float = 1e-5


def _trunc(shape, std, gen, device):
    t = torch.empty(shape, dtype=torch.float32)
    torch.nn.init.trunc_normal_(t, mean=0.0, std=std, a=-3 * std, b=3 * std, generator=gen)
    return t.to(device)


def init_params(cfg: Cfg, seed: int, device) -> dict:
    """Weights drawn like the reference's initialisers (Linear: truncated
    normal, std sqrt(2 / (in + out)); Embedding: std 1; LayerNorm gains 1),
    adaLN and lm_head included (see the module docstring); 2-D weights bf16."""
    g = torch.Generator().manual_seed(seed)

    def lin(out_f, in_f):
        return _trunc((out_f, in_f), (2 / (in_f + out_f)) ** 0.5, g, device).to(BF)

    p = {"emb": _trunc((cfg.vocab, cfg.d), 1.0, g, device).to(BF),
         "t_fc1": lin(cfg.d_cond, cfg.freq_dim), "t_fc2": lin(cfg.d_cond, cfg.d_cond),
         "freqs": torch.exp(-math.log(10000.0) * torch.arange(cfg.freq_dim // 2, dtype=torch.float32)
                            / (cfg.freq_dim // 2)).to(device),
         "layers": []}
    for _ in range(cfg.layers):
        p["layers"].append({
            "ada": lin(6 * cfg.d, cfg.d_cond), "ln1": torch.ones(cfg.d, device=device),
            "ln2": torch.ones(cfg.d, device=device), "qkv": lin(3 * cfg.d, cfg.d), "out": lin(cfg.d, cfg.d),
            "fc1": lin(cfg.d_ff, cfg.d), "fc2": lin(cfg.d, cfg.d_ff)})
    p["f_ada"] = lin(2 * cfg.d, cfg.d_cond)
    p["f_ln"] = torch.ones(cfg.d, device=device)
    p["lm_head"] = lin(cfg.vocab, cfg.d)
    return p


def linear(x, w):
    return x @ w.t()


def silu(x):
    return x * torch.sigmoid(x)


def conditioning(p, B, device):
    """c = SiLU(TimestepEmbedder(sigma = 0)) (model/modules.py:100-162, :714-716)."""
    sigma = torch.zeros(B, device=device)
    args = (sigma[:, None] * p["freqs"][None]).to(BF)
    emb = torch.cat([torch.cos(args), torch.sin(args)], dim=-1)
    return silu(silu(linear(emb, p["t_fc1"])) @ p["t_fc2"].t())


# ---------------------------------------------------------------------------
# eager backbone: the reference's ops


def ln_eager(x, w, eps):
    xf = x.float()
    num = xf - xf.mean(dim=-1, keepdim=True)
    return (w * num * torch.rsqrt(xf.var(dim=-1, keepdim=True, correction=0) + eps)).to(x.dtype)


def rope_eager(x, sin_t, cos_t, positions):
    s, c = sin_t[positions].to(x.dtype), cos_t[positions].to(x.dtype)
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], dim=-1)


def attention_eager(q, k, v, mask=None):
    scores = (q.float() @ k.float().transpose(-1, -2)) / 8.0
    if mask is not None:
        scores = torch.where(mask, scores, -torch.inf)
    probs = torch.softmax(scores, dim=-1).to(v.dtype)
    return probs @ v


def backbone_eager(cfg, p, tables, block, cache, store, mask=None):
    """cache: per layer [k, v] or None (grown with torch.cat, as KVCache).
    mask: the attention mask of a prefill pass over the whole block (the
    sampler's prompt pass, sample/sampler.py:80-87, block-causal), or None
    for a denoising step (every cached and block key visible)."""
    B, S = block.shape
    start = 0 if cache[0] is None else cache[0][0].shape[2]
    positions = torch.arange(start, start + S, device=block.device)
    x = p["emb"][block]
    c = conditioning(p, B, block.device)
    for li, L in enumerate(p["layers"]):
        sh1, sc1, g1, sh2, sc2, g2 = linear(c, L["ada"]).view(B, 6, 1, cfg.d).unbind(1)
        h = ln_eager(x, L["ln1"], cfg.eps) * (1 + sc1) + sh1
        q, k, v = linear(h, L["qkv"]).view(B, S, 3, cfg.heads, cfg.d // cfg.heads).permute(2, 0, 3, 1, 4)
        q, k = rope_eager(q, *tables, positions), rope_eager(k, *tables, positions)
        k_all, v_all = k, v
        if cache[li] is not None:
            k_all, v_all = torch.cat([cache[li][0], k], dim=2), torch.cat([cache[li][1], v], dim=2)
        if store:
            cache[li] = [k_all, v_all]
        o = attention_eager(q, k_all, v_all, mask).transpose(1, 2).reshape(B, S, cfg.d)
        x = x + g1 * linear(o, L["out"])
        h = ln_eager(x, L["ln2"], cfg.eps) * (1 + sc2) + sh2
        x = x + g2 * linear(F.gelu(linear(h, L["fc1"]), approximate="tanh"), L["fc2"])
    sh, sc = linear(c, p["f_ada"]).view(B, 2, 1, cfg.d).unbind(1)
    return linear(ln_eager(x, p["f_ln"], cfg.eps) * (1 + sc) + sh, p["lm_head"])


def sample_eager(cfg, logits, block, keep):
    """SUBS + the sampler's step (model/subs.py:11-43, sample/sampler.py:110-122)."""
    bias = torch.zeros(cfg.vocab, device=logits.device, dtype=logits.dtype)
    bias[cfg.mask] = -1e6
    x = logits + bias
    sh = x - x.amax(dim=-1, keepdim=True)
    lp = sh.float() - torch.log(torch.exp(sh.float()).sum(dim=-1, keepdim=True))
    carry = torch.full_like(lp, -1e6).scatter(-1, block.unsqueeze(-1), 0.0)
    lp = torch.where((block != cfg.mask).unsqueeze(-1), carry, lp)
    q = torch.exp(lp).double() * (1 - keep)
    q[..., cfg.mask] = keep
    u = torch.rand_like(q)
    new = torch.argmax(q / (1e-10 - torch.log(u + 1e-10)), dim=-1)
    return torch.where(block != cfg.mask, block, new)


# ---------------------------------------------------------------------------
# bd3 backbone: this library's kernels on the attention path


def ada_params(cfg, p, B, device):
    """The adaLN shift / scale / gate vectors of every block and of the
    final layer (model/modules.py:537-568, :714-716). They depend only on the
    time conditioning, which is the same for every step of a sampling run
    (sigma = 0), so the sampler computes them once per run."""
    c = conditioning(p, B, device)
    layers = [linear(c, L["ada"]).view(B, 6, 1, cfg.d).unbind(1) for L in p["layers"]]
    final = linear(c, p["f_ada"]).view(B, 2, 1, cfg.d).unbind(1)
    return layers, final


def backbone_bd3(cfg, p, tables, block, cache, store, ada=None):
    from kernels.dit_glue import gate_residual_ln_modulate, ln_modulate
    from kernels.kv_cache import attention_inputs
    B, S = block.shape
    start = cache.length
    x = p["emb"][block]
    ada_layers, ada_final = ada if ada is not None else ada_params(cfg, p, B, block.device)
    layers = p["layers"]
    sh1, sc1 = ada_layers[0][0], ada_layers[0][1]
    h = ln_modulate(x, layers[0]["ln1"], sh1, sc1, cfg.eps)
    for li, L in enumerate(layers):
        _, _, g1, sh2, sc2, g2 = ada_layers[li]
        q, k_all, v_all = attention_inputs(linear(h, L["qkv"]), cfg.heads, *tables, positions=start,
                                           kv_cache=cache, layer_idx=li, store=store)
        o = torch.ops.bd3.decode(q, k_all, v_all, cfg.bs, 0).transpose(1, 2).reshape(B, S, cfg.d)
        # each residual update fused with the LayerNorm + modulate that reads it next
        x, h = gate_residual_ln_modulate(x, g1, linear(o, L["out"]), L["ln2"], sh2, sc2, cfg.eps)
        y = linear(F.gelu(linear(h, L["fc1"]), approximate="tanh"), L["fc2"])
        if li + 1 < len(layers):
            w_next, (sh_next, sc_next) = layers[li + 1]["ln1"], ada_layers[li + 1][:2]
        else:
            w_next, (sh_next, sc_next) = p["f_ln"], ada_final
        x, h = gate_residual_ln_modulate(x, g2, y, w_next, sh_next, sc_next, cfg.eps)
    return linear(h, p["lm_head"])


def generate(cfg, p, tables, batch, n_blocks, steps, backend, check=None, graph=False):
    """sample_bd3lm with the KV cache (sample/sampler.py:37-158). `check`:
    optional callback(block_idx, step, block, caches, committed) for the logit
    check (committed: the tokens of the blocks before this one).
    graph (bd3 only): the backbone of a block's denoising steps is captured
    once per block as a HIP graph (the cache length, hence every launch
    argument, is fixed within a block) and replayed for each step; the draw
    runs outside the graph, so each step takes a fresh Philox offset."""
    from kernels.kv_cache import KVCache
    from kernels.sampling import PhiloxStream, subs_sample_step
    device = p["emb"].device
    x = torch.empty(batch, 0, device=device, dtype=torch.long)
    ada = None
    if backend == "bd3":
        cache = KVCache.empty(cfg.layers, capacity=n_blocks * cfg.bs)
        gen = PhiloxStream(seed=0)
        ada = ada_params(cfg, p, batch, device)
    else:
        cache = [None] * cfg.layers
    static_block = torch.empty((batch, cfg.bs), device=device, dtype=torch.long)
    for bi in range(n_blocks):
        block = torch.full((batch, cfg.bs), cfg.mask, device=device, dtype=torch.long)
        g_step = None
        if graph:
            static_block.copy_(block)
            if bi == 0:
                # Warm-up before the first capture (lazy library state, GEMM
                # workspaces); later blocks reuse the same shapes but the
                # cache length, which only changes kernel arguments.
                side = torch.cuda.Stream()
                side.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(side):
                    backbone_bd3(cfg, p, tables, static_block, cache, False, ada)
                torch.cuda.current_stream().wait_stream(side)
            g_step = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g_step):
                static_logits = backbone_bd3(cfg, p, tables, static_block, cache, False, ada)
        for i in range(steps):
            t, s = 1 - i / steps, 1 - (i + 1) / steps
            if check is not None:
                check(bi, i, block, cache, x)
            if backend == "bd3":
                if g_step is not None:
                    static_block.copy_(block)
                    g_step.replay()
                    logits = static_logits
                else:
                    logits = backbone_bd3(cfg, p, tables, block, cache, False, ada)
                block = subs_sample_step(logits, block, cfg.mask, s / t, generator=gen)
            else:
                logits = backbone_eager(cfg, p, tables, block, cache, False)
                block = sample_eager(cfg, logits, block, s / t)
        if backend == "bd3":
            backbone_bd3(cfg, p, tables, block, cache, True, ada)
        else:
            backbone_eager(cfg, p, tables, block, cache, True)
        x = torch.cat([x, block], dim=-1)
        del g_step
    return x


def run(blocks: int = 64, eager_blocks: int = 2, check_steps: int = 4, batch: int = 8, seed: int = 0) -> dict:
    import kernels.ops  # noqa: F401
    from kernels.kv_cache import rope_tables
    cfg = Cfg()
    device = torch.device("cuda:0")
    p = init_params(cfg, seed, device)
    tables = rope_tables(cfg.d // cfg.heads, cfg.max_seq, device=device)
    steps = cfg.bs

    # Logit check: at one denoising step of blocks spread over the run (the
    # first, the second, the middle and the last block, so the last one runs
    # against a cache of (blocks - 1) * 32 tokens), the bd3 backbone over its
    # KV cache against the eager backbone over an eager cache built
    # independently: one eager prefill pass of the committed tokens,
    # block-causal (the sampler's prompt pass, sample/sampler.py:78-87; a
    # prefill gives the same K/V as committing block by block).
    diffs = []
    check_blocks = sorted({0, 1, blocks // 2, blocks - 1} & set(range(blocks)))
    if check_steps < len(check_blocks):  # keep the last block, spread the rest
        keep = [check_blocks[round(i * (len(check_blocks) - 1) / max(check_steps - 1, 1))]
                for i in range(check_steps)] if check_steps > 1 else check_blocks[-1:]
        check_blocks = sorted(set(keep)) if check_steps else []
    check_at = {(b, steps // 2) for b in check_blocks}

    def check(bi, step, block, cache, committed):
        if (bi, step) not in check_at:
            return
        with torch.no_grad():
            eager_cache = [None] * cfg.layers
            P = committed.shape[1]
            if P:
                pos = torch.arange(P)
                causal = ((pos[None, :] // cfg.bs) <= (pos[:, None] // cfg.bs)).to(block.device)
                backbone_eager(cfg, p, tables, committed, eager_cache, True, mask=causal)
            le = backbone_eager(cfg, p, tables, block, eager_cache, False).float()
            lb = backbone_bd3(cfg, p, tables, block, cache, False).float()
            diffs.append({"block": bi, "step": step, "cache_tokens": P,
                          "max_abs": float((le - lb).abs().max()), "logit_scale": float(le.abs().max())})

    with torch.no_grad():
        generate(cfg, p, tables, batch, 1, 2, "bd3")  # warm-up
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = generate(cfg, p, tables, batch, blocks, steps, "bd3")
        torch.cuda.synchronize()
        t_bd3 = time.perf_counter() - t0
        assert not (out == cfg.mask).any(), "a [MASK] token survived the last step"
        generate(cfg, p, tables, batch, 1, 2, "bd3", graph=True)  # warm-up
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out_g = generate(cfg, p, tables, batch, blocks, steps, "bd3", graph=True)
        torch.cuda.synchronize()
        t_graph = time.perf_counter() - t0
        # same weights, same Philox stream: replayed graphs draw the same tokens
        graph_equal = bool(torch.equal(out, out_g))
        generate(cfg, p, tables, batch, blocks, steps, "bd3", check=check)
        generate(cfg, p, tables, batch, 1, 2, "eager")  # warm-up
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        generate(cfg, p, tables, batch, eager_blocks, steps, "eager")
        torch.cuda.synchronize()
        t_eager = time.perf_counter() - t0
    return {
        "workload": f"configs[4]: {batch} x {blocks * cfg.bs} tokens, blocks of {cfg.bs}, {steps} steps per block, "
                    f"12L / 768 / 12H, vocab 50258, KV cache, bf16 weights (random init, seed {seed})",
        "tokens_per_s": batch * blocks * cfg.bs / t_graph,
        "seconds": t_graph,
        "launch": "hip_graph per block (backbone), eager draw",
        "eager_launch_tokens_per_s": batch * blocks * cfg.bs / t_bd3,
        "graph_tokens_equal_eager_launch": graph_equal,
        "reference_eager_tokens_per_s": batch * eager_blocks * cfg.bs / t_eager,
        "reference_eager_blocks": eager_blocks,
        "logit_check": diffs,
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--blocks", type=int, default=64)
    ap.add_argument("--eager-blocks", type=int, default=2)
    ap.add_argument("--check-steps", type=int, default=4)
    args = ap.parse_args(argv)
    print(json.dumps(run(args.blocks, args.eager_blocks, args.check_steps)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
