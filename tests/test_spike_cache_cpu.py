"""Cache layout and metadata conventions, on the CPU (no kernel launches).

Known answers: spikeinfer/engine/spike_cache.py:66-69 (3,072 B per token for the
24-layer, T=4, H_kv=2, head_dim 64 model), tests/test_cpu_backend.py:184-190 (slot
matrix), engine/spike_cache.py:83-88 (last block reserved for padding).
"""
from __future__ import annotations

import pytest
import torch

from spikeinfer_amd.attention import AttentionMetadata, paged_attention
from spikeinfer_amd.spike_cache import PagedSpikeCache, slot_mapping


def test_bytes_per_token_known_answer():
    per_block = PagedSpikeCache.bytes_per_block(24, 4, 2, 64, 16)
    assert per_block // 16 == 3072


def test_layout_and_pad_block():
    c = PagedSpikeCache(2, 4, 2, 64, num_blocks=10, block_size=16, device="cpu")
    assert len(c.layers) == 2
    assert tuple(c.k[0].shape) == (4, 2, 160, 2) and c.k[0].dtype == torch.int32
    assert int(c.k[1].abs().sum()) == 0
    assert c.pad_block == 9 and c.pad_slot == 144
    assert c.num_allocatable_blocks == 9 and c.capacity_tokens == 144
    assert c.nbytes == 2 * 2 * 4 * 2 * 160 * 2 * 4
    c.v[1].fill_(5)
    c.reset()
    assert int(c.v[1].abs().sum()) == 0


@pytest.mark.parametrize("blocks,bs", [(1, 16), (4, 12)])
def test_rejects_bad_geometry(blocks, bs):
    with pytest.raises(ValueError):
        PagedSpikeCache(1, 4, 2, 64, num_blocks=blocks, block_size=bs, device="cpu")


def test_slot_matrix_known_answer():
    tables = [[3, 1, 7], [5, 2, 0]]
    got = [slot_mapping(t, 0, 10, 4) for t in tables]
    assert got == [[12, 13, 14, 15, 4, 5, 6, 7, 28, 29], [20, 21, 22, 23, 8, 9, 10, 11, 0, 1]]
    assert slot_mapping(tables[0], 9, 1, 4) == [29]


def test_metadata_counts_prefill_chunks():
    meta = AttentionMetadata(slot_mapping=torch.arange(3), block_size=16, num_decode_tokens=3,
                             block_tables=torch.zeros(3, 2, dtype=torch.int32),
                             seq_lens=torch.ones(3, dtype=torch.int32))
    assert meta.num_prefills == 0
    meta.prefill_query_lens.append(5)
    assert meta.num_prefills == 1


def test_paged_attention_refuses_cpu_tensors():
    """The product path has no CPU fallback: CPU tensors are an error."""
    c = PagedSpikeCache(1, 4, 2, 64, num_blocks=4, block_size=16, device="cpu")
    meta = AttentionMetadata(slot_mapping=torch.tensor([0]), block_size=16)
    spk = torch.zeros(4, 1, 2, 1, 64)
    with pytest.raises(ValueError, match="GPU"):
        paged_attention(torch.zeros(4, 1, 14, 1, 64), spk, spk, c.k[0], c.v[0], meta, 14, 2, 64)


def test_attention_metadata_on_device():
    """AttentionMetadata.on (spikeinfer/attention.py:62-95): the object itself
    when its tensors are already on the device; otherwise one copy per device,
    made once, with every index tensor moved and the plain fields shared."""
    import torch
    from spikeinfer_amd.attention import AttentionMetadata

    meta = AttentionMetadata(slot_mapping=torch.arange(5), block_size=16, num_decode_tokens=2,
                             block_tables=torch.zeros((2, 3), dtype=torch.int32),
                             seq_lens=torch.tensor([3, 7], dtype=torch.int32),
                             prefill_query_starts=[2], prefill_query_lens=[3], prefill_context_lens=[0],
                             prefill_block_tables=[torch.tensor([4], dtype=torch.int32)])
    assert meta.on(torch.device("cpu")) is meta
    assert meta.on("cpu") is meta
    moved = meta.on("meta")
    assert moved is not meta and meta.on(torch.device("meta")) is moved
    assert moved.slot_mapping.device.type == "meta" and moved.block_tables.device.type == "meta"
    assert moved.seq_lens.device.type == "meta" and moved.prefill_block_tables[0].device.type == "meta"
    assert (moved.block_size, moved.num_decode_tokens, moved.prefill_query_lens) == (16, 2, [3])
    assert moved.on("meta") is moved
    assert meta.slot_mapping.device.type == "cpu"  # the original is untouched
