"""Seeded synthetic inputs shared by the CPU and GPU tests (numpy only).

Shapes and conventions follow the reference tests: scrambled physical blocks
(tests/test_spike_attention.py:38-46), pad-block padded tables
(tests/test_cpu_backend.py:266-305), Bernoulli spike bits packed little-endian.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as orc


def random_bits(rng, shape, density):
    return (rng.random(shape) < density).astype(np.uint8)


def attn_case(seq_lens, block_size=16, T=4, q_heads=14, kv_heads=2, head_dim=64,
              density=0.4, q_density=0.4, seed=0, extra_blocks=3, compact=False):
    """Packed q/k/v, a scrambled block table padded with the pad block, lens.

    ``compact`` sizes the cache to the blocks the sequences use (many short
    sequences beside one long one) instead of n * max_blocks."""
    rng = np.random.default_rng(seed)
    n = len(seq_lens)
    max_blocks = max(1, max((s + block_size - 1) // block_size for s in seq_lens))
    used = sum((s + block_size - 1) // block_size for s in seq_lens)
    num_blocks = (used if compact else n * max_blocks) + extra_blocks
    slots = num_blocks * block_size
    k = orc.pack(random_bits(rng, (T, kv_heads, slots, head_dim), density))
    v = orc.pack(random_bits(rng, (T, kv_heads, slots, head_dim), density))
    q = orc.pack(random_bits(rng, (T, n, q_heads, head_dim), q_density))
    order = rng.permutation(num_blocks - 1)
    tables = np.full((n, max_blocks), num_blocks - 1, dtype=np.int32)
    cur = 0
    for i, s in enumerate(seq_lens):
        need = (s + block_size - 1) // block_size
        tables[i, :need] = order[cur:cur + need]
        cur += need
    return dict(q=q, k=k, v=v, tables=tables, lens=np.asarray(seq_lens, np.int32),
                head_dim=head_dim, block_size=block_size, num_q_heads=q_heads,
                num_kv_heads=kv_heads)


def oracle_attn(case):
    c = case
    return orc.decode_attn(c["q"], c["k"], c["v"], c["tables"], c["lens"], c["head_dim"],
                           c["block_size"], c["num_q_heads"], c["num_kv_heads"])
