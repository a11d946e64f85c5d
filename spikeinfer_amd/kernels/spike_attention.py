"""Paged popcount decode attention on gfx950 (drop-in for
spikeinfer/kernels/spike_attention.py:153-244).

The HIP kernel serves all ``num_q_heads // num_kv_heads`` query heads of a KV
head from one read of the KV blocks, scores with ``v_bcnt``, and uses the fixed
softmax offset ``popcount(q)`` (an upper bound of every integer score), so long
contexts split into partitions whose partial sums simply add.
"""
from __future__ import annotations

import functools
import math

import torch

from .. import _lib
from .packing import packed_width


def _as_int32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 else t.to(torch.int32)


def _check_packed(name: str, t: torch.Tensor) -> None:
    if t.dtype != torch.int32:
        raise ValueError(f"{name} must be int32 packed words, got {t.dtype}")
    if t.ndim != 4 or t.stride(-1) != 1:
        raise ValueError(f"{name} must be 4-D with a contiguous word axis")


@functools.lru_cache(maxsize=256)
def decode_attn_workspace_bytes(
    T: int, n_seqs: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
    block_size: int, max_blocks: int,
) -> int:
    """Scratch bytes :func:`paged_spike_attn_decode` needs for this shape
    (a pure function of the shape: cached, so eager calls skip the query)."""
    return int(
        _lib.load().spk_decode_attn_workspace_bytes(
            T, n_seqs, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks
        )
    )


def paged_spike_attn_decode(
    q_packed: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    head_dim: int,
    block_size: int,
    num_q_heads: int,
    num_kv_heads: int,
    out: torch.Tensor | None = None,
    dtype: torch.dtype = torch.float32,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """One decode step of attention against the paged spike cache.

    Same contract as the reference (spike_attention.py:153-189): ``q_packed``
    ``int32 [T, N, H_q, W]``, caches ``int32 [T, H_kv, num_slots, W]``,
    ``block_tables int32 [N, max_blocks]``, ``seq_lens int32 [N]`` including
    the token being decoded; ``out`` optional ``[T, N, H_q, head_dim]`` (needed
    for graph capture).  ``workspace`` optionally supplies the partition
    scratch (``uint8``, at least :func:`decode_attn_workspace_bytes`); by
    default it comes from torch's caching allocator, which is capture-safe.
    """
    T, n_seqs, n_heads, words = q_packed.shape
    if words != packed_width(head_dim):
        raise ValueError(f"q has {words} words, expected {packed_width(head_dim)}")
    if n_heads != num_q_heads:
        raise ValueError(f"q has {n_heads} heads, expected {num_q_heads}")
    dev = _lib.require_gpu(q_packed, k_cache, v_cache, block_tables, seq_lens, out)
    _check_packed("q_packed", q_packed)
    _check_packed("k_cache", k_cache)
    _check_packed("v_cache", v_cache)
    if k_cache.shape != v_cache.shape:
        raise ValueError(f"k/v cache shapes differ: {tuple(k_cache.shape)} vs {tuple(v_cache.shape)}")
    if k_cache.shape[1] != num_kv_heads or k_cache.shape[0] != T or k_cache.shape[3] != words:
        raise ValueError(
            f"cache shape {tuple(k_cache.shape)} does not match T={T}, H_kv={num_kv_heads}, W={words}"
        )
    block_tables = _as_int32(block_tables)
    seq_lens = _as_int32(seq_lens).contiguous()
    if block_tables.ndim != 2 or block_tables.shape[0] < n_seqs or seq_lens.numel() < n_seqs:
        raise ValueError("block_tables must be [N, max_blocks] and seq_lens [N]")

    if out is None:
        out = torch.empty((T, n_seqs, n_heads, head_dim), device=dev, dtype=dtype)
    elif tuple(out.shape) != (T, n_seqs, n_heads, head_dim):
        raise ValueError(f"out has shape {tuple(out.shape)}, expected {(T, n_seqs, n_heads, head_dim)}")
    if n_seqs == 0:
        return out

    max_blocks = block_tables.shape[1]
    need = decode_attn_workspace_bytes(
        T, n_seqs, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks
    )
    if need:
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=dev)
        elif workspace.numel() * workspace.element_size() < need:
            raise ValueError(f"workspace holds {workspace.nbytes} bytes, need {need}")
    ws_ptr = workspace.data_ptr() if (need and workspace is not None) else None

    _lib.check(
        _lib.load().spk_decode_attn(
            q_packed.data_ptr(), _lib.strides(q_packed),
            k_cache.data_ptr(), _lib.strides(k_cache),
            v_cache.data_ptr(), _lib.strides(v_cache), k_cache.shape[2],
            block_tables.data_ptr(), block_tables.stride(0), block_tables.stride(1),
            seq_lens.data_ptr(), out.data_ptr(), _lib.dtype_code(out.dtype), _lib.strides(out),
            T, n_seqs, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks,
            1.0 / math.sqrt(head_dim), ws_ptr, need, _lib.stream_of(dev),
        ),
        "paged_spike_attn_decode",
    )
    return out


def paged_spike_attn_scores(
    q_packed: torch.Tensor,
    k_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    head_dim: int,
    block_size: int,
    num_q_heads: int,
    num_kv_heads: int,
    max_len: int,
) -> torch.Tensor:
    """Integer scores ``popcount(q & k)`` as ``int32 [T, N, H_q, max_len]``
    (positions at or past ``seq_len`` hold -1), through the same block-table
    walk as the decode kernel.  Exposed to check the score path bit-exactly.
    """
    T, n_seqs, n_heads, words = q_packed.shape
    if words != packed_width(head_dim) or n_heads != num_q_heads:
        raise ValueError("q_packed does not match head_dim / num_q_heads")
    dev = _lib.require_gpu(q_packed, k_cache, block_tables, seq_lens)
    _check_packed("q_packed", q_packed)
    _check_packed("k_cache", k_cache)
    block_tables = _as_int32(block_tables)
    seq_lens = _as_int32(seq_lens).contiguous()
    scores = torch.full((T, n_seqs, n_heads, max_len), -1, dtype=torch.int32, device=dev)
    _lib.check(
        _lib.load().spk_decode_scores(
            q_packed.data_ptr(), _lib.strides(q_packed), k_cache.data_ptr(), _lib.strides(k_cache),
            k_cache.shape[2], block_tables.data_ptr(), block_tables.stride(0),
            block_tables.stride(1), seq_lens.data_ptr(), scores.data_ptr(), max_len,
            T, n_seqs, num_q_heads, num_kv_heads, head_dim, block_size, _lib.stream_of(dev),
        ),
        "paged_spike_attn_scores",
    )
    return scores


def _gather(k_cache, v_cache, block_table, seq_len, head_dim, block_size, dtype):
    dev = _lib.require_gpu(k_cache, v_cache, block_table)
    _check_packed("cache", k_cache)
    if v_cache is not None and (v_cache.shape != k_cache.shape or v_cache.stride() != k_cache.stride()):
        raise ValueError("k and v caches must have the same shape and strides")
    if k_cache.shape[-1] != packed_width(head_dim):
        raise ValueError(f"cache has {k_cache.shape[-1]} words, expected {packed_width(head_dim)}")
    T, H = k_cache.shape[0], k_cache.shape[1]
    table = _as_int32(block_table)
    if table.ndim != 1:
        raise ValueError("block_table must be one sequence's 1-D row")
    target = torch.uint8 if dtype == torch.bool else dtype
    k_out = torch.empty((T, H, seq_len, head_dim), dtype=target, device=dev)
    v_out = torch.empty_like(k_out) if v_cache is not None else None
    _lib.check(
        _lib.load().spk_gather_unpack(
            k_cache.data_ptr(), _lib.ptr(v_cache), _lib.strides(k_cache), k_cache.shape[2],
            table.data_ptr(), table.stride(0), table.numel(), seq_len, k_out.data_ptr(),
            _lib.ptr(v_out), _lib.dtype_code(target), T, H, head_dim, block_size,
            _lib.stream_of(dev),
        ),
        "gather_kv_unpacked",
    )
    if dtype == torch.bool:
        k_out = k_out.view(torch.bool)
        v_out = v_out.view(torch.bool) if v_out is not None else None
    return k_out, v_out


def gather_kv_unpacked(
    cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_len: int,
    head_dim: int,
    block_size: int,
    dtype: torch.dtype,
) -> torch.Tensor:
    """One sequence's first ``seq_len`` cached tokens as dense ``[T, H_kv, S, D]``
    0/1 spikes (the prefill reader, spike_attention.py:224-244), in one HIP
    launch: block-table walk and unpack together, no packed temporary."""
    return _gather(cache, None, block_table, seq_len, head_dim, block_size, dtype)[0]


def gather_kv_unpacked_pair(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_len: int,
    head_dim: int,
    block_size: int,
    dtype: torch.dtype,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``gather_kv_unpacked`` of the K and the V cache in one launch."""
    return _gather(k_cache, v_cache, block_table, seq_len, head_dim, block_size, dtype)


def paged_spike_attn_decode_partials(
    q_packed: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    head_dim: int,
    block_size: int,
    num_q_heads: int,
    num_kv_heads: int,
    part_len: int,
    partials: torch.Tensor | None = None,
) -> torch.Tensor:
    """Unnormalised per-partition sums of the decode attention:
    ``float32 [P, T, N, H_q, head_dim + 1]`` with ``P = ceil(max_blocks *
    block_size / part_len)``; entry ``[p, t, n, h, :head_dim]`` is
    ``sum_j w_j v_j`` and ``[..., head_dim]`` is ``sum_j w_j`` over the
    tokens ``j`` of partition ``p`` (``w_j = exp(-popcount(q & ~k_j) /
    sqrt(head_dim))``, the fixed softmax offset, so partials of any split add).
    Partitions at or past a sequence's length are left unwritten.  Finish with
    :func:`combine_partitions`."""
    T, n_seqs, n_heads, words = q_packed.shape
    if words != packed_width(head_dim) or n_heads != num_q_heads:
        raise ValueError("q_packed does not match head_dim / num_q_heads")
    dev = _lib.require_gpu(q_packed, k_cache, v_cache, block_tables, seq_lens, partials)
    for name, t in (("q_packed", q_packed), ("k_cache", k_cache), ("v_cache", v_cache)):
        _check_packed(name, t)
    if part_len <= 0 or part_len % block_size:
        raise ValueError(f"part_len={part_len} must be a positive multiple of block_size={block_size}")
    block_tables = _as_int32(block_tables)
    seq_lens = _as_int32(seq_lens).contiguous()
    max_blocks = block_tables.shape[1]
    P = -(-max_blocks * block_size // part_len)
    shape = (P, T, n_seqs, num_q_heads, head_dim + 1)
    if partials is None:
        partials = torch.empty(shape, dtype=torch.float32, device=dev)
    elif tuple(partials.shape) != shape or partials.dtype != torch.float32 or not partials.is_contiguous():
        raise ValueError(f"partials must be contiguous float32 {shape}")
    if n_seqs == 0:
        return partials
    _lib.check(
        _lib.load().spk_decode_attn_partials(
            q_packed.data_ptr(), _lib.strides(q_packed), k_cache.data_ptr(), _lib.strides(k_cache),
            v_cache.data_ptr(), _lib.strides(v_cache), k_cache.shape[2], block_tables.data_ptr(),
            block_tables.stride(0), block_tables.stride(1), seq_lens.data_ptr(), T, n_seqs,
            num_q_heads, num_kv_heads, head_dim, block_size, max_blocks,
            1.0 / math.sqrt(head_dim), part_len, partials.data_ptr(),
            partials.numel() * 4, _lib.stream_of(dev),
        ),
        "paged_spike_attn_decode_partials",
    )
    return partials


def combine_partitions(
    partials: torch.Tensor,
    seq_lens: torch.Tensor,
    part_len: int,
    out: torch.Tensor | None = None,
    dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """``[P, T, N, H_q, D + 1]`` partials -> ``[T, N, H_q, D]`` attention
    output: for each row, the sums over partitions ``p < ceil(seq_len /
    part_len)`` in partition order, ``out = sum a / sum l`` (zeros for
    ``seq_len <= 0``)."""
    if partials.ndim != 5 or partials.dtype != torch.float32 or not partials.is_contiguous():
        raise ValueError("partials must be contiguous float32 [P, T, N, H_q, D + 1]")
    P, T, n_seqs, n_heads, d1 = partials.shape
    dev = _lib.require_gpu(partials, seq_lens, out)
    seq_lens = _as_int32(seq_lens).contiguous()
    if out is None:
        out = torch.empty((T, n_seqs, n_heads, d1 - 1), dtype=dtype, device=dev)
    elif tuple(out.shape) != (T, n_seqs, n_heads, d1 - 1):
        raise ValueError(f"out has shape {tuple(out.shape)}, expected {(T, n_seqs, n_heads, d1 - 1)}")
    _lib.check(
        _lib.load().spk_decode_attn_combine(
            partials.data_ptr(), partials.numel() * 4, P, part_len, seq_lens.data_ptr(), out.data_ptr(),
            _lib.dtype_code(out.dtype), _lib.strides(out), T, n_seqs, n_heads, d1 - 1,
            _lib.stream_of(dev),
        ),
        "combine_partitions",
    )
    return out
