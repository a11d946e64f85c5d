"""Torch-eager restatements of the reference's non-kernel paths.

``spikeinfer/kernels/__init__.py:1-29`` exports three functions that are not
GPU kernels: ``lif_multistep_ref`` (the recurrence in eager torch,
``lif_triton.py:126-138``), ``paged_spike_attn_decode_ref`` (per-sequence
unpack + SDPA, ``spike_attention.py:247-282``) and
``paged_spike_attn_decode_cpu`` (the grouped CPU strategy,
``spike_attention_cpu.py:66-222``).  This module gives the same three, written
for this package in plain torch so they run on any device, and with them a
torch pack and unpack (``pack_spikes_torch``, ``unpack_spikes_torch``, the
reference's CPU packing) that do not need the HIP library.

They are separate, explicitly named entry points.  The HIP operators in
``spike_attention.py`` and ``lif.py`` never call into this module: a CPU
tensor handed to them raises instead of falling back here.
"""
from __future__ import annotations

import os

import torch
import torch.nn.functional as F

from .packing import BITS_PER_WORD, packed_width

# Unpacked K+V bytes the grouped CPU path holds at once (the reference's
# measured cache-fitting size, spike_attention_cpu.py:66-75); overridable with
# SPIKEINFER_CPU_GATHER_BUDGET_MB.
CPU_GATHER_BUDGET = 16 << 20


def unpack_spikes_torch(words: torch.Tensor, num_channels: int,
                        dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``int32 [..., W]`` -> ``[..., num_channels]`` 0/1 with shifts and masks
    (bit i of word w is channel 32w + i), on whatever device ``words`` is."""
    W = packed_width(num_channels)
    if words.shape[-1] != W:
        raise ValueError(f"expected {W} words for {num_channels} channels, got {words.shape[-1]}")
    shifts = torch.arange(BITS_PER_WORD, device=words.device, dtype=torch.int32)
    bits = (words.to(torch.int32).unsqueeze(-1) >> shifts) & 1  # [..., W, 32]
    bits = bits.reshape(*words.shape[:-1], W * BITS_PER_WORD)[..., :num_channels]
    return bits.to(dtype)


def pack_spikes_torch(x: torch.Tensor) -> torch.Tensor:
    """``[..., C]`` (nonzero = spike) -> ``int32 [..., ceil(C/32)]`` with tensor
    ops, the reference's CPU packing (packing.py:97-111): bits shifted into
    place and summed per 32-channel word, values >= 2^31 wrapped to negative
    int32; tail bits zero."""
    C = x.shape[-1]
    W = packed_width(C)
    bits = (x != 0).to(torch.int64)
    if W * BITS_PER_WORD != C:
        bits = F.pad(bits, (0, W * BITS_PER_WORD - C))
    bits = bits.reshape(*bits.shape[:-1], W, BITS_PER_WORD)
    shifts = torch.arange(BITS_PER_WORD, device=x.device, dtype=torch.int64)
    acc = (bits << shifts).sum(dim=-1)
    acc = torch.where(acc >= 2 ** 31, acc - 2 ** 32, acc)
    return acc.to(torch.int32)


def lif_multistep_ref(x, beta, threshold, mem0=None, out_dtype=None):
    """The LIF recurrence in eager torch (lif_triton.py:126-138): for each t,
    ``r = (u - th > 0)``, ``u = beta*u + x_t - r*th``, ``s_t = (u - th > 0)``,
    fp32, beta clamped to [0, 1].  Returns ``(spikes, u_final)``."""
    b = beta.clamp(0, 1).to(torch.float32)
    th = threshold.to(torch.float32)
    if mem0 is None:
        u = torch.zeros(x.shape[1:], dtype=torch.float32, device=x.device)
    else:
        u = mem0.to(torch.float32).clone()
    spikes = torch.empty(x.shape, dtype=out_dtype or x.dtype, device=x.device)
    for t in range(x.shape[0]):
        fired = (u - th > 0).to(torch.float32)
        u = b * u + x[t].to(torch.float32) - fired * th
        spikes[t] = (u - th > 0).to(spikes.dtype)
    return spikes, u


def _slots_of(block_tables: torch.Tensor, length: int, block_size: int) -> torch.Tensor:
    """``[n, max_blocks]`` tables -> ``int64 [n, length]`` cache slots
    (slot = table[p // bs] * bs + p % bs, block_manager.py:71-77)."""
    pos = torch.arange(length, device=block_tables.device, dtype=torch.int64)
    blk = block_tables.to(torch.int64).index_select(1, pos // block_size)
    return blk * block_size + pos % block_size


def _gather(cache, slots, num_channels):
    """Cache ``[T, H, slots, W]`` at ``slots [n, S]`` -> dense fp32
    ``[T, n, H, S, D]`` (the gather runs on packed words, then one unpack)."""
    T, H = cache.shape[0], cache.shape[1]
    n, S = slots.shape
    words = cache.index_select(2, slots.reshape(-1)).view(T, H, n, S, -1).transpose(1, 2)
    return unpack_spikes_torch(words, num_channels, torch.float32)


def paged_spike_attn_decode_ref(q_packed, k_cache, v_cache, block_tables, seq_lens, head_dim,
                                block_size, num_q_heads, num_kv_heads, dtype=torch.float32):
    """One sequence at a time: unpack q and the sequence's first ``seq_len``
    cached tokens, repeat the kv heads to the query heads, SDPA with the
    default 1/sqrt(head_dim) scale (spike_attention.py:247-282)."""
    T, N = q_packed.shape[0], q_packed.shape[1]
    rep = num_q_heads // num_kv_heads
    out = torch.empty((T, N, num_q_heads, head_dim), dtype=dtype, device=q_packed.device)
    for i in range(N):
        L = int(seq_lens[i])
        slots = _slots_of(block_tables[i:i + 1], L, block_size)
        k = _gather(k_cache, slots, head_dim)[:, 0]  # [T, H_kv, L, D]
        v = _gather(v_cache, slots, head_dim)[:, 0]
        if rep > 1:
            k = k.repeat_interleave(rep, dim=1)
            v = v.repeat_interleave(rep, dim=1)
        q = unpack_spikes_torch(q_packed[:, i], head_dim, torch.float32).unsqueeze(2)
        out[:, i] = F.scaled_dot_product_attention(q, k, v).squeeze(2).to(dtype)
    return out


def paged_spike_attn_decode_cpu(q_packed, k_cache, v_cache, block_tables, seq_lens, head_dim,
                                block_size, num_q_heads, num_kv_heads, out=None,
                                dtype=torch.float32):
    """The reference's CPU strategy (spike_attention_cpu.py:103-222): runs of
    consecutive sequences whose unpacked K+V (padded to the run's longest)
    fit the gather budget share one slot-matrix gather, one unpack and one
    SDPA call with ``enable_gqa``; a -inf mask is built only when the run's
    lengths differ.  Same signature as ``paged_spike_attn_decode``."""
    T, N, Hq = q_packed.shape[0], q_packed.shape[1], q_packed.shape[2]
    if out is None:
        out = torch.empty((T, N, Hq, head_dim), dtype=dtype, device=q_packed.device)
    env = os.environ.get("SPIKEINFER_CPU_GATHER_BUDGET_MB")
    budget = max(1, int(float(env) * (1 << 20))) if env else CPU_GATHER_BUDGET
    per_token = T * num_kv_heads * head_dim * 4 * 2  # fp32 K and V
    lens = [int(x) for x in seq_lens.tolist()]
    i = 0
    while i < N:
        j, longest = i + 1, lens[i]
        while j < N and (j + 1 - i) * max(longest, lens[j]) * per_token <= budget:
            longest = max(longest, lens[j])
            j += 1
        run = lens[i:j]
        slots = _slots_of(block_tables[i:j], longest, block_size)
        n = j - i
        k = _gather(k_cache, slots, head_dim).reshape(T * n, num_kv_heads, longest, head_dim)
        v = _gather(v_cache, slots, head_dim).reshape(T * n, num_kv_heads, longest, head_dim)
        q = unpack_spikes_torch(q_packed[:, i:j], head_dim, torch.float32)
        q = q.reshape(T * n, Hq, 1, head_dim)
        mask = None
        if any(L != longest for L in run):
            keep = torch.arange(longest, device=q.device)[None, :] < torch.tensor(run, device=q.device)[:, None]
            mask = torch.zeros((n, longest), dtype=torch.float32, device=q.device)
            mask.masked_fill_(~keep, float("-inf"))
            mask = mask[None, :, None, None, :].expand(T, n, 1, 1, longest).reshape(T * n, 1, 1, longest)
        ctx = F.scaled_dot_product_attention(q, k, v, attn_mask=mask,
                                             enable_gqa=num_q_heads != num_kv_heads)
        out[:, i:j].copy_(ctx.view(T, n, Hq, head_dim).to(out.dtype))
        i = j
    return out
