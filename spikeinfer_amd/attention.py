"""Attention against the paged spike cache (counterpart of spikeinfer/attention.py).

``paged_attention`` keeps the reference's contract (spikeinfer/attention.py:111-180):
dense 0/1 spikes in, the step's K/V packed and scattered into the cache at
``meta.slot_mapping`` first, decode tokens (a contiguous prefix of the batch) through
the popcount decode kernel, prefill chunks through unpack-gather + SDPA with a causal
mask offset by the cached prefix, output ``[T, 1, n_tok, H_q * D]`` in the spikes'
dtype.

``paged_attention_fused`` is the same step starting one stage earlier, from the LIF
input currents: the fused LIF -> pack -> cache-write kernel replaces
``lif_multistep`` + ``pack_spikes`` + ``index_copy_`` for K and V (and LIF + pack for
the decode queries), so dense q/k/v spikes are never materialised for decode tokens.
"""
from __future__ import annotations

from dataclasses import dataclass, field, replace

import torch
import torch.nn.functional as F

from .kernels.lif import lif_multistep, lif_pack_write_sites
from .kernels.packing import pack_spikes, packed_width
from .kernels.spike_attention import gather_kv_unpacked_pair, paged_spike_attn_decode


@dataclass
class AttentionMetadata:
    """Per-step batch description consumed by the attention operators.

    Field names are the engine's contract (spikeinfer/attention.py:33-95).
    Tokens are ordered decodes first: rows ``[0, num_decode_tokens)`` are one
    decode token per sequence, described by ``block_tables``/``seq_lens``;
    the rest are prefill chunks described by the four ``prefill_*`` lists.
    """

    slot_mapping: torch.Tensor  # int64 [n_tok]: cache slot each token's K/V bits go to
    block_size: int
    num_decode_tokens: int = 0
    # int32 [n_dec, max_blocks]; unused entries hold the cache's pad block
    block_tables: torch.Tensor | None = None
    # int32 [n_dec]; counts the token being decoded (its K/V is written first)
    seq_lens: torch.Tensor | None = None
    # chunk i covers batch rows [starts[i], starts[i] + query_lens[i]) and sits
    # after context_lens[i] already-cached positions of its sequence
    prefill_query_starts: list[int] = field(default_factory=list)
    prefill_query_lens: list[int] = field(default_factory=list)
    prefill_context_lens: list[int] = field(default_factory=list)
    prefill_block_tables: list[torch.Tensor] = field(default_factory=list)

    # device -> copy of this metadata there (see on()); not part of equality
    _copies: dict = field(default_factory=dict, repr=False, compare=False)

    @property
    def num_prefills(self) -> int:
        return len(self.prefill_query_lens)

    def on(self, device: torch.device | str) -> "AttentionMetadata":
        """The same metadata with its index tensors on ``device``
        (spikeinfer/attention.py:62-95): ``self`` when ``slot_mapping`` is
        already there, otherwise a copy made once per device and kept on this
        object (metadata is rebuilt every step, so the copies live one step)."""
        device = torch.device(device)
        if self.slot_mapping.device == device:
            return self
        key = str(device)
        if key not in self._copies:
            move = lambda t: None if t is None else t.to(device, non_blocking=True)
            self._copies[key] = replace(
                self, slot_mapping=move(self.slot_mapping), block_tables=move(self.block_tables),
                seq_lens=move(self.seq_lens),
                prefill_block_tables=[move(t) for t in self.prefill_block_tables], _copies={})
        return self._copies[key]


def _causal_offset_mask(query_len: int, total_len: int, device, dtype) -> torch.Tensor:
    """Additive mask letting query i (at position total_len - query_len + i)
    see positions <= its own (spikeinfer/attention.py:320-330)."""
    ctx = total_len - query_len
    mask = torch.full((query_len, total_len), float("-inf"), device=device, dtype=dtype)
    return torch.triu(mask, diagonal=ctx + 1)


def _prefill(q_dense, k_cache, v_cache, meta, out, num_q_heads, num_kv_heads, head_dim):
    """Each prefill chunk attends to its sequence's whole cached prefix plus
    itself: one gather-unpack launch yields dense K and V, then SDPA with the
    offset causal mask (spikeinfer/attention.py:161-178)."""
    dtype, device = q_dense.dtype, q_dense.device
    for i in range(meta.num_prefills):
        start = meta.prefill_query_starts[i]
        q_len = meta.prefill_query_lens[i]
        total = meta.prefill_context_lens[i] + q_len
        table = meta.prefill_block_tables[i]
        k_all, v_all = gather_kv_unpacked_pair(k_cache, v_cache, table, total, head_dim,
                                               meta.block_size, dtype)
        q = q_dense[:, :, start:start + q_len, :]  # [T, H_q, q_len, D]
        o = F.scaled_dot_product_attention(
            q, k_all, v_all,
            attn_mask=_causal_offset_mask(q_len, total, device, dtype),
            enable_gqa=num_q_heads != num_kv_heads,
        )
        out[:, start:start + q_len] = o.permute(0, 2, 1, 3)


def paged_attention(
    q_spk: torch.Tensor,
    k_spk: torch.Tensor,
    v_spk: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    meta: AttentionMetadata,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
) -> torch.Tensor:
    """Spike attention over the paged cache, reference signature.

    ``q_spk, k_spk, v_spk``: ``[T, 1, H, n_tok, D]`` 0/1 spikes; caches ``int32
    [T, H_kv, num_slots, W]`` of this layer.  Returns ``[T, 1, n_tok, H_q * D]``.
    """
    T, n_tok = q_spk.shape[0], q_spk.shape[3]
    dtype, device = q_spk.dtype, q_spk.device
    k_cache.index_copy_(2, meta.slot_mapping, pack_spikes(k_spk.squeeze(1)))
    v_cache.index_copy_(2, meta.slot_mapping, pack_spikes(v_spk.squeeze(1)))
    out = torch.empty((T, n_tok, num_q_heads, head_dim), device=device, dtype=dtype)
    n_dec = meta.num_decode_tokens
    if n_dec:
        q_dec = q_spk[:, 0, :, :n_dec, :].permute(0, 2, 1, 3)  # [T, n_dec, H_q, D]
        paged_spike_attn_decode(
            pack_spikes(q_dec), k_cache, v_cache, meta.block_tables, meta.seq_lens,
            head_dim=head_dim, block_size=meta.block_size, num_q_heads=num_q_heads,
            num_kv_heads=num_kv_heads, out=out[:, :n_dec],
        )
    if meta.num_prefills:
        _prefill(q_spk[:, 0], k_cache, v_cache, meta, out, num_q_heads, num_kv_heads, head_dim)
    return out.view(T, 1, n_tok, num_q_heads * head_dim)


def paged_attention_fused(
    q_cur: torch.Tensor,
    k_cur: torch.Tensor,
    v_cur: torch.Tensor,
    lif_q: tuple[torch.Tensor, torch.Tensor],
    lif_k: tuple[torch.Tensor, torch.Tensor],
    lif_v: tuple[torch.Tensor, torch.Tensor],
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    meta: AttentionMetadata,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    out: torch.Tensor | None = None,
    q_packed: torch.Tensor | None = None,
) -> torch.Tensor:
    """One attention step from the LIF input currents.

    Equivalent to running the three LIF sites (``lif_multistep`` with per-head_dim
    ``(beta, threshold)``, spikeinfer/modeling_fast.py:132-134) and then
    ``paged_attention``, but the K/V spikes go straight from the LIF kernel into
    their cache slots and decode queries straight into a packed buffer.

    Args:
        q_cur, k_cur, v_cur: ``[T, n_tok, H, D]`` currents (any strides, e.g.
            ``proj_out.view(T, n_tok, H, D)`` of the projection + RoPE output).
        lif_q, lif_k, lif_v: ``(beta, threshold)`` of each site, ``[D]`` each.
        out: optional preallocated ``[T, n_tok, H_q, D]`` in the currents' dtype.
        q_packed: optional preallocated ``int32 [T, n_dec, H_q, W]`` buffer.
        Both are needed for graph capture (stable addresses).

    Returns ``[T, 1, n_tok, H_q * D]`` in ``q_cur.dtype``.
    """
    T, n_tok = q_cur.shape[0], q_cur.shape[1]
    dtype, device = q_cur.dtype, q_cur.device
    if out is None:
        out = torch.empty((T, n_tok, num_q_heads, head_dim), device=device, dtype=dtype)
    n_dec = meta.num_decode_tokens
    # One launch for the three LIF sites: k and v into their cache slots, the
    # decode tokens' q into the packed-query buffer.
    sites = [(k_cur, lif_k[0], lif_k[1], k_cache, True), (v_cur, lif_v[0], lif_v[1], v_cache, True)]
    if n_dec:
        if q_packed is None:
            q_packed = torch.empty((T, n_dec, num_q_heads, packed_width(head_dim)),
                                   dtype=torch.int32, device=device)
        sites.append((q_cur[:, :n_dec], lif_q[0], lif_q[1], q_packed, False))
    lif_pack_write_sites(sites, meta.slot_mapping)
    if n_dec:
        paged_spike_attn_decode(
            q_packed, k_cache, v_cache, meta.block_tables, meta.seq_lens,
            head_dim=head_dim, block_size=meta.block_size, num_q_heads=num_q_heads,
            num_kv_heads=num_kv_heads, out=out[:, :n_dec],
        )
    if meta.num_prefills:
        # Prefill queries need dense spikes for SDPA; the LIF is per token, so
        # running it on the prefill tokens alone gives the same spikes.
        q_pre = lif_multistep(q_cur[:, n_dec:], lif_q[0], lif_q[1])  # [T, n_pre, H_q, D]
        q_dense = torch.zeros((T, num_q_heads, n_tok, head_dim), device=device, dtype=dtype)
        q_dense[:, :, n_dec:] = q_pre.permute(0, 2, 1, 3)
        _prefill(q_dense, k_cache, v_cache, meta, out, num_q_heads, num_kv_heads, head_dim)
    return out.view(T, 1, n_tok, num_q_heads * head_dim)
