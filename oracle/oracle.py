"""numpy front end of the C oracle, plus pure-numpy / pure-Python twins.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Every function names the
reference code it restates.  The twins are independent formulations used to
pin the C restatement (tests/test_oracle.py):
  * np_pack / np_unpack use numpy.packbits(bitorder="little"), the layout
    spikeinfer/kernels/packing.py:16-23 specifies;
  * np_lif steps the recurrence with numpy float32 scalars-per-op, the same
    per-operation rounding as torch eager (lif_triton.py:126-138);
  * brute_attn evaluates textbook softmax attention in Python floats on the
    unpacked bits, like the SDPA oracle spike_attention.py:247-282.
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np

from . import build as _build

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_build.LIB):
            _build.build()
        _lib = ctypes.CDLL(_build.LIB)
        P = ctypes.c_void_p
        I, L = ctypes.c_int, ctypes.c_int64
        _lib.orc_threads.argtypes = [I]
        _lib.orc_threads.restype = I
        _lib.orc_pack_rows.argtypes = [P, L, I, P]
        _lib.orc_unpack_rows.argtypes = [P, L, I, P]
        _lib.orc_lif.argtypes = [P, I, L, I, P, P, P, P, P]
        _lib.orc_decode_attn.argtypes = [P, P, P, P, P, I, I, I, I, I, I, L, L, P]
        _lib.orc_decode_scores.argtypes = [P, P, P, P, I, I, I, I, I, I, L, L, I, P]
        _lib.orc_lif_pack_write.argtypes = [P, I, L, I, I, P, P, P, P, L]
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def threads(n: int = 0) -> int:
    """Sets (n > 0) and returns the OpenMP thread count of the C oracle."""
    return lib().orc_threads(n)


def packed_width(c: int) -> int:
    return (c + 31) // 32


# ---- packing ---------------------------------------------------------------
def pack(bits: np.ndarray) -> np.ndarray:
    """[..., C] nonzero -> int32 [..., W] (C oracle)."""
    C = bits.shape[-1]
    b = np.ascontiguousarray(bits != 0, dtype=np.uint8).reshape(-1, C)
    out = np.empty((b.shape[0], packed_width(C)), dtype=np.int32)
    lib().orc_pack_rows(_p(b), b.shape[0], C, _p(out))
    return out.reshape(*bits.shape[:-1], packed_width(C))


def unpack(words: np.ndarray, C: int) -> np.ndarray:
    w = np.ascontiguousarray(words, dtype=np.int32).reshape(-1, words.shape[-1])
    out = np.empty((w.shape[0], C), dtype=np.uint8)
    lib().orc_unpack_rows(_p(w), w.shape[0], C, _p(out))
    return out.reshape(*words.shape[:-1], C)


def np_pack(bits: np.ndarray) -> np.ndarray:
    """Independent twin: numpy.packbits little-endian, padded to 32 bits."""
    C = bits.shape[-1]
    W = packed_width(C)
    b = (np.asarray(bits) != 0).astype(np.uint8)
    pad = W * 32 - C
    if pad:
        b = np.concatenate([b, np.zeros(b.shape[:-1] + (pad,), np.uint8)], axis=-1)
    by = np.packbits(b, axis=-1, bitorder="little")
    return np.ascontiguousarray(by).view("<i4")


def np_unpack(words: np.ndarray, C: int) -> np.ndarray:
    by = np.ascontiguousarray(words, dtype="<i4").view(np.uint8)
    return np.unpackbits(by, axis=-1, bitorder="little")[..., :C]


# ---- LIF -------------------------------------------------------------------
def lif(x: np.ndarray, beta: np.ndarray, thr: np.ndarray, mem0: np.ndarray | None = None):
    """x float32 [T, ..., N] -> (spikes uint8 same shape, final u float32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, N = x.shape[0], x.shape[-1]
    M = x.size // (T * N)
    spk = np.empty(x.shape, np.uint8)
    u = np.empty(x.shape[1:], np.float32)
    m0 = None if mem0 is None else np.ascontiguousarray(mem0, np.float32)
    lib().orc_lif(_p(x), T, M, N, _p(np.ascontiguousarray(beta, np.float32)),
                  _p(np.ascontiguousarray(thr, np.float32)), _p(m0), _p(spk), _p(u))
    return spk, u


def np_lif(x: np.ndarray, beta: np.ndarray, thr: np.ndarray, mem0=None):
    """Independent twin in numpy float32 (one rounding per operation)."""
    x = np.asarray(x, np.float32)
    b = np.clip(np.asarray(beta, np.float32), np.float32(0), np.float32(1))
    th = np.asarray(thr, np.float32)
    u = np.zeros(x.shape[1:], np.float32) if mem0 is None else np.array(mem0, np.float32)
    spk = np.empty(x.shape, np.uint8)
    for t in range(x.shape[0]):
        r = ((u - th) > 0).astype(np.float32)
        u = (b * u + x[t]) - r * th
        spk[t] = (u - th) > 0
    return spk, u


def lif_pack_write(x, beta, thr, out, slots=None):
    """x float32 [T, n_tok, H, D]; packs into out (packed buffer or cache)."""
    x = np.ascontiguousarray(x, np.float32)
    T, n_tok, H, D = x.shape
    S = out.shape[2] if slots is not None else 0
    sl = None if slots is None else np.ascontiguousarray(slots, np.int64)
    assert out.flags.c_contiguous and out.dtype == np.int32
    lib().orc_lif_pack_write(_p(x), T, n_tok, H, D, _p(np.ascontiguousarray(beta, np.float32)),
                             _p(np.ascontiguousarray(thr, np.float32)), _p(out), _p(sl), S)
    return out


# ---- attention -------------------------------------------------------------
def decode_attn(q, k, v, tables, lens, head_dim, block_size, num_q_heads, num_kv_heads):
    """C oracle: float64 [T, N, Hq, D] (spike_attention.py:86-150 semantics)."""
    q = np.ascontiguousarray(q, np.int32)
    k = np.ascontiguousarray(k, np.int32)
    v = np.ascontiguousarray(v, np.int32)
    tables = np.ascontiguousarray(tables, np.int32)
    lens = np.ascontiguousarray(lens, np.int32)
    T, N = q.shape[0], q.shape[1]
    out = np.empty((T, N, num_q_heads, head_dim), np.float64)
    lib().orc_decode_attn(_p(q), _p(k), _p(v), _p(tables), _p(lens), T, N, num_q_heads,
                          num_kv_heads, head_dim, block_size, tables.shape[1], k.shape[2],
                          _p(out))
    return out


def decode_scores(q, k, tables, lens, head_dim, block_size, num_q_heads, num_kv_heads, max_len):
    q = np.ascontiguousarray(q, np.int32)
    k = np.ascontiguousarray(k, np.int32)
    tables = np.ascontiguousarray(tables, np.int32)
    lens = np.ascontiguousarray(lens, np.int32)
    T, N = q.shape[0], q.shape[1]
    out = np.empty((T, N, num_q_heads, max_len), np.int32)
    lib().orc_decode_scores(_p(q), _p(k), _p(tables), _p(lens), T, N, num_q_heads, num_kv_heads,
                            head_dim, block_size, tables.shape[1], k.shape[2], max_len, _p(out))
    return out


def brute_attn(q, k, v, tables, lens, head_dim, block_size, num_q_heads, num_kv_heads):
    """Pure-Python twin for tiny inputs: unpack, dot products, textbook
    softmax (no max subtraction needed at these magnitudes), weighted mean."""
    T, N = q.shape[0], q.shape[1]
    nrep = num_q_heads // num_kv_heads
    scale = 1.0 / math.sqrt(head_dim)
    qb, kb, vb = np_unpack(q, head_dim), np_unpack(k, head_dim), np_unpack(v, head_dim)
    out = np.zeros((T, N, num_q_heads, head_dim))
    for t in range(T):
        for n in range(N):
            L = int(lens[n])
            slots = [int(tables[n][p // block_size]) * block_size + p % block_size for p in range(L)]
            for h in range(num_q_heads):
                kvh = h // nrep
                s = [sum(int(a) * int(b) for a, b in zip(qb[t, n, h], kb[t, kvh, sl])) * scale
                     for sl in slots]
                e = [math.exp(x) for x in s]
                z = sum(e)
                for d in range(head_dim):
                    out[t, n, h, d] = sum(e[j] * int(vb[t, kvh, slots[j], d]) for j in range(L)) / z
    return out


def prefill_attn(q_bits, k_cache, v_cache, table, context_len, head_dim, block_size,
                 num_q_heads, num_kv_heads):
    """One prefill chunk (spikeinfer/attention.py:161-178): ``q_bits`` 0/1
    ``[T, Hq, q_len, D]`` at positions ``[context_len, context_len + q_len)``,
    attending causally to the sequence's cached positions ``[0, context_len +
    q_len)`` read through ``table`` (slot = table[p // bs] * bs + p % bs,
    block_manager.py:71-77).  Float64 textbook softmax over the unpacked bits,
    max-subtracted; returns ``[T, Hq, q_len, D]``."""
    T, _, q_len, _ = q_bits.shape
    total = context_len + q_len
    nrep = num_q_heads // num_kv_heads
    pos = np.arange(total)
    slots = np.asarray(table, np.int64)[pos // block_size] * block_size + pos % block_size
    kb = np_unpack(k_cache[:, :, slots], head_dim).astype(np.float64)  # [T, Hkv, total, D]
    vb = np_unpack(v_cache[:, :, slots], head_dim).astype(np.float64)
    kb = np.repeat(kb, nrep, axis=1)
    vb = np.repeat(vb, nrep, axis=1)
    s = np.einsum("thqd,thkd->thqk", q_bits.astype(np.float64), kb) / math.sqrt(head_dim)
    visible = pos[None, :] <= (context_len + np.arange(q_len))[:, None]  # [q_len, total]
    s = np.where(visible, s, -np.inf)
    s -= s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    return np.einsum("thqk,thkd->thqd", e, vb) / e.sum(axis=-1, keepdims=True)


# ---- sampling ----------------------------------------------------------------
def sample_row(logits, temperature=1.0, top_k=-1, top_p=1.0, min_p=0.0, rep=1.0,
               presence=0.0, frequency=0.0, history=(), u=0.0):
    """One row of spikeinfer/engine/sampler.py:48-177 in numpy.

    Penalties in float32 over the generated tokens (:98-119: repetition
    ``v / r if v > 0 else v * r``, then ``v - (presence + frequency * count)``),
    ``x = v / temperature`` in float32 (:69-75), then in float64: min_p on the
    softmax (:137-141), top_k on the descending order (:143-153), top_p on the
    mass strictly before each token (:155-159).  Equal values are ordered by
    index (a stable sort; the reference leaves it to torch.topk).  The draw
    walks the kept tokens in the same order (value descending, index
    ascending) and takes the first whose inclusive cumulative probability
    exceeds ``u``.

    Returns (token, kept bool mask, kept probabilities, margin, order):
    ``margin`` is the smallest distance of a filter cut (min_p, top_p) from its
    decision boundary -- below ~1e-6 the float32 kernel may legitimately
    decide the other way; ``order`` lists the kept tokens in draw order (the
    cumulative sums of ``probs[order]`` are the draw's boundaries).
    """
    v = np.asarray(logits, np.float32).copy()
    counts = {}
    for t in history:
        counts[int(t)] = counts.get(int(t), 0) + 1
    for t, c in counts.items():
        if rep != 1.0:
            v[t] = v[t] / np.float32(rep) if v[t] > 0 else v[t] * np.float32(rep)
        if presence or frequency:
            v[t] = v[t] - (np.float32(presence) + np.float32(frequency) * np.float32(c))
    V = v.shape[0]
    if temperature < 1e-5:
        tok = int(np.argmax(v))
        kept = np.zeros(V, bool)
        kept[tok] = True
        return tok, kept, kept.astype(np.float64), np.inf, np.array([tok])
    x = (v / np.float32(temperature)).astype(np.float32)
    m = float(x.max())
    w = np.exp(x.astype(np.float64) - m)
    margin = np.inf
    alive = np.ones(V, bool)
    if min_p > 0:
        alive = w >= min_p
        margin = min(margin, float(np.min(np.abs(w - min_p))))
    order = np.lexsort((np.arange(V), -x.astype(np.float64)))  # value desc, index asc
    order = order[alive[order]]
    if 0 < top_k < len(order):
        order = order[:top_k]
    if top_p < 1.0:
        p = w[order] / w[order].sum()
        before = np.cumsum(p) - p
        keep = before < top_p
        margin = min(margin, float(np.min(np.abs(before - top_p))))
        order = order[keep]
    kept = np.zeros(V, bool)
    kept[order] = True
    probs = np.where(kept, w, 0.0)
    probs /= probs.sum()
    cdf = np.cumsum(probs[order])
    pos = min(int(np.searchsorted(cdf, u, side="right")), len(order) - 1)
    return int(order[pos]), kept, probs, margin, order
