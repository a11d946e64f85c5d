"""The paged packed spike KV cache (counterpart of spikeinfer/engine/spike_cache.py:20-101).

Per layer two ``int32 [T, H_kv, num_blocks * block_size, W]`` slabs, keys and
values, zero-initialised; ``W = ceil(head_dim / 32)`` words per (t, head, slot)
with bit ``i`` of word ``w`` = channel ``32w + i``.  A block is ``block_size``
consecutive slots, so one block of one (t, head) is ``block_size * 4W`` contiguous
bytes (128 B at block size 16, head_dim 64) -- the unit the decode kernel reads.

The last block is reserved (never handed out): captured decode batches are padded to
a bucket size, and their padding rows write their K/V to this block and attend with
``seq_len = 1`` against it (spikeinfer/engine/model_runner.py:234-240).
"""
from __future__ import annotations

import torch

from .kernels.packing import packed_width


class PagedSpikeCache:
    def __init__(
        self,
        num_layers: int,
        timesteps: int,
        num_kv_heads: int,
        head_dim: int,
        num_blocks: int,
        block_size: int,
        device: str | torch.device = "cuda",
    ) -> None:
        if num_blocks < 2:
            raise ValueError("need at least 2 blocks (one is reserved for padding)")
        if block_size <= 0 or block_size & (block_size - 1):
            raise ValueError(f"block_size={block_size} must be a power of two")
        self.num_layers = num_layers
        self.timesteps = timesteps
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.words = packed_width(head_dim)
        shape = (timesteps, num_kv_heads, num_blocks * block_size, self.words)
        dev = torch.device(device)
        self.k = [torch.zeros(shape, dtype=torch.int32, device=dev) for _ in range(num_layers)]
        self.v = [torch.zeros(shape, dtype=torch.int32, device=dev) for _ in range(num_layers)]
        self.layers = list(zip(self.k, self.v))

    @staticmethod
    def bytes_per_block(
        num_layers: int, timesteps: int, num_kv_heads: int, head_dim: int, block_size: int
    ) -> int:
        return 2 * num_layers * timesteps * num_kv_heads * block_size * packed_width(head_dim) * 4

    @property
    def nbytes(self) -> int:
        return self.bytes_per_block(
            self.num_layers, self.timesteps, self.num_kv_heads, self.head_dim, self.block_size
        ) * self.num_blocks

    @property
    def num_allocatable_blocks(self) -> int:
        return self.num_blocks - 1

    @property
    def pad_block(self) -> int:
        return self.num_blocks - 1

    @property
    def pad_slot(self) -> int:
        return self.pad_block * self.block_size

    @property
    def capacity_tokens(self) -> int:
        return self.num_allocatable_blocks * self.block_size

    def reset(self) -> None:
        for t in self.k + self.v:
            t.zero_()


def slot_mapping(block_table: list[int], start: int, count: int, block_size: int) -> list[int]:
    """Physical slots of logical positions ``[start, start + count)``
    (spikeinfer/engine/block_manager.py:71-77): block_table[p // bs] * bs + p % bs."""
    return [block_table[p // block_size] * block_size + p % block_size for p in range(start, start + count)]
