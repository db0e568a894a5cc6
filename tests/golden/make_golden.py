"""Generate tests/golden/bd3_golden.json: brute-force known answers for tiny
shapes, computed with plain Python loops straight from the reference's
written rules (no numpy, no torch), independent of the oracle's vectorised
code.

    python tests/golden/make_golden.py

Contents:
  train_masks   block_diff_mask for small (n, bs), from the rule list in the
                docstring of model/bd3lm.py:17-21 ("noisy q, block b -> noisy
                keys in block b; noisy q, block b -> clean keys in blocks < b;
                clean q, block b -> clean keys in blocks <= b"), as row strings.
  decode_masks  the decode rule of kernels/BlockSparseDecodeAttention.py:84-88
                and :23-26 for small (q_len, kv_len, bs).
  attention     softmax(q k^T / sqrt(d) + M) v and the natural-log LSE per row
                (model/modules.py:738-771; kernels/BlockSparseFlashAttention.py:169)
                for one tiny training case, in double precision with math.exp,
                on small exactly representable inputs.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

OUT = Path(__file__).with_name("bd3_golden.json")


def rule_mask(n: int, bs: int) -> list[str]:
    rows = []
    for q in range(2 * n):
        row = []
        for k in range(2 * n):
            q_noisy, k_noisy = q < n, k < n
            qb = (q if q_noisy else q - n) // bs
            kb = (k if k_noisy else k - n) // bs
            if q_noisy and k_noisy:
                live = qb == kb
            elif q_noisy and not k_noisy:
                live = kb < qb
            elif not q_noisy and not k_noisy:
                live = kb <= qb
            else:
                live = False
            row.append("1" if live else "0")
        rows.append("".join(row))
    return rows


def rule_decode_mask(q_len: int, kv_len: int, bs: int) -> list[str]:
    rows = []
    for i in range(q_len):
        pos = kv_len - q_len + i
        rows.append("".join("1" if (j // bs) <= (pos // bs) else "0" for j in range(kv_len)))
    return rows


def lcg_values(count: int, seed: int) -> list[float]:
    """Small multiples of 1/8 in [-1, 1]: exact in bf16 and fp32."""
    out, s = [], seed
    for _ in range(count):
        s = (1103515245 * s + 12345) % (1 << 31)
        out.append(((s >> 16) % 17 - 8) / 8.0)
    return out


def brute_attention(n: int, bs: int, d: int, seed: int) -> dict:
    S = 2 * n
    q = lcg_values(S * d, seed)
    k = lcg_values(S * d, seed + 1)
    v = lcg_values(S * d, seed + 2)
    mask = rule_mask(n, bs)
    scale = 1.0 / math.sqrt(d)
    out, lse = [], []
    for i in range(S):
        logits = []
        for j in range(S):
            if mask[i][j] == "1":
                s = sum(q[i * d + t] * k[j * d + t] for t in range(d)) * scale
                logits.append((j, s))
        m = max(s for _, s in logits)
        z = sum(math.exp(s - m) for _, s in logits)
        lse.append(m + math.log(z))
        row = [0.0] * d
        for j, s in logits:
            p = math.exp(s - m) / z
            for t in range(d):
                row[t] += p * v[j * d + t]
        out.extend(row)
    return {"n": n, "block_size": bs, "d": d, "q": q, "k": k, "v": v, "out": out, "lse": lse}


def main() -> None:
    golden = {
        "train_masks": [
            {"n": n, "block_size": bs, "rows": rule_mask(n, bs)}
            for n, bs in [(1, 1), (2, 1), (4, 1), (4, 2), (4, 4), (6, 2), (6, 3), (6, 4), (8, 2),
                          (8, 8), (12, 5)]
        ],
        "decode_masks": [
            {"q_len": ql, "kv_len": kl, "block_size": bs, "rows": rule_decode_mask(ql, kl, bs)}
            for ql, kl, bs in [(1, 1, 1), (2, 6, 2), (4, 4, 2), (3, 10, 4), (6, 9, 3), (5, 5, 8)]
        ],
        "attention": [brute_attention(4, 2, 4, 11), brute_attention(6, 3, 8, 5)],
    }
    OUT.write_text(json.dumps(golden, indent=None, separators=(",", ":")) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
