"""Writes the golden fixtures in this folder (run: python tests/golden/make_golden.py).

Every expected value comes from the independent pure-numpy / pure-Python twins
in oracle/oracle.py (np_pack, np_unpack, np_lif, brute_attn) on seeded inputs,
not from the C oracle or the HIP kernels, which the fixtures then check.  No
reference code is imported or run.

  config1_attn.npz   config 1 of the baseline: N=1, Hq 14 / Hkv 2, head_dim 64,
                     T=4, ctx 128, block_size 16, scrambled block table,
                     Bernoulli(0.2) q/k/v bits (spike_attention.py:67-150).
  lif_boundary.npz   membrane hovering at threshold (tests/test_lif_kernel.py:
                     192-210 scenario, M reduced from 256 to 32 to keep the file
                     small): spikes and final membrane, two roundings per step.
  hand_cases.json    known answers quoted from the reference's tests.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as orc  # noqa: E402


def config1():
    rng = np.random.default_rng(1000)
    T, Hq, Hkv, D, bs, ctx = 4, 14, 2, 64, 16, 128
    num_blocks = 12  # 8 used + 3 spare + the pad block
    slots = num_blocks * bs
    bits = lambda shape: (rng.random(shape) < 0.2).astype(np.uint8)
    k = orc.np_pack(bits((T, Hkv, slots, D)))
    v = orc.np_pack(bits((T, Hkv, slots, D)))
    q = orc.np_pack(bits((T, 1, Hq, D)))
    tables = np.full((1, 8), num_blocks - 1, np.int32)
    tables[0] = rng.permutation(num_blocks - 1)[:8]
    lens = np.array([ctx], np.int32)
    out = orc.brute_attn(q, k, v, tables, lens, D, bs, Hq, Hkv)
    pos = np.arange(ctx)
    sl = tables[0][pos // bs] * bs + pos % bs
    qb = orc.np_unpack(q, D).astype(np.int64)  # [T, 1, Hq, D]
    kb = orc.np_unpack(k[:, :, sl], D).astype(np.int64)  # [T, Hkv, ctx, D]
    kb = np.repeat(kb, Hq // Hkv, axis=1)
    scores = np.einsum("thd,thpd->thp", qb[:, 0], kb).astype(np.int32)[:, None]
    np.savez_compressed(os.path.join(HERE, "config1_attn.npz"), q=q, k=k, v=v, tables=tables,
                        lens=lens, scores=scores, out=out)


def lif_boundary():
    rng = np.random.default_rng(0)
    T, M, N = 8, 32, 64
    beta = np.full(N, 0.9, np.float32)
    thr = np.full(N, 1.0, np.float32)
    x = (np.ones((T, M, N)) + rng.standard_normal((T, M, N)) * 1e-6).astype(np.float32)
    spikes, u = orc.np_lif(x, beta, thr)
    np.savez_compressed(os.path.join(HERE, "lif_boundary.npz"), x=x, beta=beta, thr=thr,
                        spikes_packed=np.packbits(spikes, axis=-1, bitorder="little"), u=u)


def hand_cases():
    cases = {
        "lif_constant_current": {
            "cite": "beta 0.9, threshold 1.0, I = 1.0: u_0 = 1.0 sits on the threshold",
            "beta": 0.9, "threshold": 1.0, "current": 1.0, "T": 4, "spikes": [0, 1, 1, 1],
        },
        "pack_all_ones": {"cite": "tests/test_packing.py:45-50", "channels": 64,
                          "words": [-1, -1]},
        "pack_c33_tail": {"cite": "tests/test_packing.py:66-70", "channels": 33,
                          "words": [-1, 1]},
        "pack_single_channel": {"cite": "tests/test_packing.py:53-63", "channels": 64,
                                "set": [0, 31, 32, 63],
                                "words": [[1, 0], [-2147483648, 0], [0, 1], [0, -2147483648]]},
        "slot_matrix": {"cite": "tests/test_cpu_backend.py:184-190", "block_size": 4,
                        "tables": [[3, 1, 7], [5, 2, 0]], "len": 10,
                        "slots": [[12, 13, 14, 15, 4, 5, 6, 7, 28, 29],
                                  [20, 21, 22, 23, 8, 9, 10, 11, 0, 1]]},
        "bytes_per_token": {"cite": "engine/spike_cache.py:66-69", "layers": 24, "T": 4,
                            "kv_heads": 2, "head_dim": 64, "bytes": 3072},
    }
    # Self-check against the numpy twins before writing.
    for name in ("pack_all_ones", "pack_c33_tail"):
        c = cases[name]
        assert orc.np_pack(np.ones((1, c["channels"]), np.uint8))[0].tolist() == c["words"]
    c = cases["pack_single_channel"]
    for ch, w in zip(c["set"], c["words"]):
        b = np.zeros((1, 64), np.uint8)
        b[0, ch] = 1
        assert orc.np_pack(b)[0].tolist() == w
    c = cases["lif_constant_current"]
    s, _ = orc.np_lif(np.full((4, 1, 1), 1.0, np.float32), np.array([0.9], np.float32),
                      np.array([1.0], np.float32))
    assert s[:, 0, 0].tolist() == c["spikes"]
    with open(os.path.join(HERE, "hand_cases.json"), "w") as f:
        json.dump(cases, f, indent=1)


if __name__ == "__main__":
    config1()
    lif_boundary()
    hand_cases()
    print("fixtures written to", HERE)
