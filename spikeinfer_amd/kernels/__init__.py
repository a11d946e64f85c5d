"""Public kernel API, mirroring spikeinfer/kernels/__init__.py:1-29.

Every function here launches HIP kernels on gfx950 through the C ABI in
include/spikeinfer_amd.h; none has a CPU fallback.
"""
from .lif import lif_multistep, lif_pack_write, validate_thresholds
from .packing import (
    BITS_PER_WORD,
    pack_spikes,
    packed_bytes_per_token,
    packed_width,
    unpack_spikes,
)
from .spike_attention import (
    decode_attn_workspace_bytes,
    gather_kv_unpacked,
    paged_spike_attn_decode,
    paged_spike_attn_scores,
)

__all__ = [
    "lif_multistep",
    "lif_pack_write",
    "validate_thresholds",
    "pack_spikes",
    "unpack_spikes",
    "packed_width",
    "packed_bytes_per_token",
    "BITS_PER_WORD",
    "paged_spike_attn_decode",
    "paged_spike_attn_scores",
    "decode_attn_workspace_bytes",
    "gather_kv_unpacked",
]
