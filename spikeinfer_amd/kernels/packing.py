"""Bit layout and pack/unpack of spike tensors on gfx950.

Layout (same as spikeinfer/kernels/packing.py:16-23): bit ``i`` of int32 word
``w`` is channel ``32*w + i``, words ascending along the channel axis.  On a
little-endian machine the two int32 words of a head_dim-64 vector are byte for
byte one uint64 whose bit ``c`` is channel ``c``.
"""
from __future__ import annotations

import torch

from .. import _lib

BITS_PER_WORD = 32

_PACKABLE = (torch.float32, torch.float16, torch.bfloat16, torch.uint8, torch.int32)


def packed_width(num_channels: int) -> int:
    """Words needed to hold ``num_channels`` spikes (packing.py:46-48)."""
    return (num_channels + BITS_PER_WORD - 1) // BITS_PER_WORD


def packed_bytes_per_token(
    num_layers: int, num_timesteps: int, num_kv_heads: int, head_dim: int
) -> int:
    """KV bytes one cached token costs, K and V, whole model (packing.py:155-159)."""
    return 2 * num_layers * num_timesteps * num_kv_heads * packed_width(head_dim) * 4


def pack_spikes(x: torch.Tensor) -> torch.Tensor:
    """``[..., C]`` -> ``int32 [..., ceil(C/32)]``; nonzero packs as 1.

    Mirrors pack_spikes (packing.py:84-111); one HIP launch (one wave per row,
    one ``__ballot`` per 64 channels).
    """
    dev = _lib.require_gpu(x)
    channels = x.shape[-1]
    words = packed_width(channels)
    if x.dtype == torch.bool:
        x = x.view(torch.uint8)
    elif x.dtype not in _PACKABLE:
        x = (x != 0).to(torch.uint8)
    flat = x.reshape(-1, channels)
    if channels > 1 and flat.stride(1) != 1:
        flat = flat.contiguous()
    rows = flat.shape[0]
    out = torch.empty((rows, words), dtype=torch.int32, device=dev)
    row_stride = flat.stride(0) if rows > 1 else channels
    _lib.check(
        _lib.load().spk_pack(
            flat.data_ptr(), _lib.dtype_code(flat.dtype), row_stride, out.data_ptr(),
            rows, channels, _lib.stream_of(dev),
        ),
        "pack_spikes",
    )
    return out.view(*x.shape[:-1], words)


def unpack_spikes(
    words: torch.Tensor, num_channels: int, dtype: torch.dtype = torch.float32
) -> torch.Tensor:
    """``int32 [..., W]`` -> ``[..., num_channels]`` of 0/1 in ``dtype``.

    Mirrors unpack_spikes (packing.py:136-152), including its ValueError.
    """
    expected = packed_width(num_channels)
    if words.shape[-1] != expected:
        raise ValueError(
            f"expected {expected} words for {num_channels} channels, got {words.shape[-1]}"
        )
    dev = _lib.require_gpu(words)
    if words.dtype != torch.int32:
        raise ValueError(f"packed words must be int32, got {words.dtype}")
    flat = words.reshape(-1, expected).contiguous()
    rows = flat.shape[0]
    target = torch.uint8 if dtype == torch.bool else dtype
    out = torch.empty((rows, num_channels), dtype=target, device=dev)
    _lib.check(
        _lib.load().spk_unpack(
            flat.data_ptr(), rows, num_channels, out.data_ptr(), _lib.dtype_code(target),
            _lib.stream_of(dev),
        ),
        "unpack_spikes",
    )
    if dtype == torch.bool:
        out = out.view(torch.bool)
    return out.view(*words.shape[:-1], num_channels)
