"""Public kernel API, mirroring spikeinfer/kernels/__init__.py:1-29.

The operators launch HIP kernels on gfx950 through the C ABI in
include/spikeinfer_amd.h and have no CPU fallback.  The ``*_ref`` /
``*_cpu`` names (reference_paths.py) are the reference's eager-torch paths,
restated; the operators never call them.
"""
from .lif import lif_multistep, lif_pack_write, lif_pack_write_sites, validate_thresholds
from .packing import (
    BITS_PER_WORD,
    pack_spikes,
    packed_bytes_per_token,
    packed_width,
    unpack_spikes,
)
from .reference_paths import (
    lif_multistep_ref,
    pack_spikes_torch,
    paged_spike_attn_decode_cpu,
    paged_spike_attn_decode_ref,
    unpack_spikes_torch,
)
from .spike_attention import (
    combine_partitions,
    decode_attn_workspace_bytes,
    gather_kv_unpacked,
    gather_kv_unpacked_pair,
    paged_spike_attn_decode_partials,
    paged_spike_attn_decode,
    paged_spike_attn_scores,
)

__all__ = [
    "lif_multistep",
    "lif_multistep_ref",
    "paged_spike_attn_decode_ref",
    "paged_spike_attn_decode_cpu",
    "unpack_spikes_torch",
    "pack_spikes_torch",
    "lif_pack_write",
    "lif_pack_write_sites",
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
    "gather_kv_unpacked_pair",
    "paged_spike_attn_decode_partials",
    "combine_partitions",
]
