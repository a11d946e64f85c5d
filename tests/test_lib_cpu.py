"""The C-ABI library loads, exports every symbol the header declares, and
rejects bad arguments on the host -- no kernel is launched (CPU only)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from spikeinfer_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "spikeinfer_amd.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(spk_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert _declared() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.spk_abi_version() == _lib.ABI_VERSION


def _i64(*v):
    return (ctypes.c_int64 * len(v))(*v)


def test_host_side_validation_without_a_gpu():
    lib = _lib.load()
    s4 = _i64(0, 0, 0, 1)
    rc = lib.spk_decode_attn(None, s4, None, s4, None, s4, 0, None, 0, 0, None, None, 0, s4,
                             4, 1, 5, 2, 64, 16, 8, 0.125, None, 0, None)
    assert rc == _lib.SPK_EINVAL and b"multiple" in lib.spk_last_error()
    rc = lib.spk_decode_attn(None, s4, None, s4, None, s4, 0, None, 0, 0, None, None, 0, s4,
                             4, 1, 14, 2, 64, 24, 8, 0.125, None, 0, None)
    assert rc == _lib.SPK_EINVAL and b"power of two" in lib.spk_last_error()
    rc = lib.spk_decode_attn(None, s4, None, s4, None, s4, 0, None, 0, 0, None, None, 0, s4,
                             4, 1, 14, 2, 256, 16, 8, 0.0625, None, 0, None)
    assert rc == _lib.SPK_EUNSUPPORTED
    rc = lib.spk_decode_attn(None, s4, None, s4, None, s4, 0, None, 0, 0, None, None, 0, s4,
                             4, 1, 14, 2, 64, 16, 8, 5.0, None, 0, None)
    assert rc == _lib.SPK_EINVAL and b"scale" in lib.spk_last_error()
    # split contexts (past 32768 tokens) need a workspace; a missing one is
    # rejected, not faulted
    rc = lib.spk_decode_attn(None, s4, None, s4, None, s4, 0, None, 0, 0, None, None, 0, s4,
                             4, 8, 14, 2, 64, 16, 4096, 0.125, None, 0, None)
    assert rc == _lib.SPK_EINVAL and b"workspace" in lib.spk_last_error()
    assert lib.spk_lif_multistep(None, 2, _i64(0, 0, 1), None, None, 0, None, None, 0, None,
                                 0, 4, 4, None) == _lib.SPK_EINVAL
    assert lib.spk_lif_pack_write(None, 2, _i64(0, 0, 0, 1), None, None, 0, None, _i64(0, 0, 0),
                                  None, 0, None, 0, 4, 4, 2, 256, None) == _lib.SPK_EUNSUPPORTED
    assert lib.spk_pack(None, 9, 1, None, 4, 4, None) == _lib.SPK_EINVAL
    sites = bytes(ctypes.sizeof(_lib.SpkLifSite) * 5)
    assert lib.spk_lif_pack_write_sites(sites, 5, 2, 4, None, None) == _lib.SPK_EINVAL
    assert lib.spk_lif_pack_write_sites(sites, 0, 2, 4, None, None) == _lib.SPK_EINVAL
    one = _lib.pack_lif_site(0, (0, 0, 0, 1), 0, 0, 0, 1, 0, (0, 0, 1), 0, 3, 2, 64)
    assert lib.spk_lif_pack_write_sites(one, 1, 2, 4, None, None) == _lib.SPK_EINVAL
    assert b"slot_mapping" in lib.spk_last_error()


def test_packed_site_bytes_match_the_c_struct():
    """pack_lif_site's bytes are the SpkLifSite layout of the header (as
    ctypes lays it out under the platform ABI)."""
    raw = _lib.pack_lif_site(1, (2, 3, 4, 5), 6, 7, 8, 9, 10, (11, 12, 13), 14, 15, 16, 17)
    assert len(raw) == ctypes.sizeof(_lib.SpkLifSite) == 120
    st = _lib.SpkLifSite.from_buffer_copy(raw)
    assert (st.x, list(st.x_strides), st.beta, st.threshold, st.param_dtype, st.scatter, st.out,
            list(st.out_strides), st.num_slots, st.n_tok, st.H, st.D) == (
        1, [2, 3, 4, 5], 6, 7, 8, 9, 10, [11, 12, 13], 14, 15, 16, 17)


def test_decode_gemm_entry_points_validate_on_the_host():
    """The decode GEMM entry points reject unsupported or malformed calls
    before any launch (fake pointers are never dereferenced)."""
    lib = _lib.load()
    bf16, f16, f32 = 2, 1, 0
    A, B = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x1001)  # 16-byte aligned / not
    assert lib.spk_linear_pack(None, 20, 896, bf16, None, None) == _lib.SPK_EINVAL
    assert lib.spk_linear_pack(None, 896, 896, f16, None, None) == _lib.SPK_EUNSUPPORTED
    assert lib.spk_linear_decode(A, A, None, A, 8, 896, 896, f16, None) == _lib.SPK_EUNSUPPORTED
    assert lib.spk_linear_decode(A, A, None, A, 300, 896, 896, bf16, None) == _lib.SPK_EUNSUPPORTED
    assert lib.spk_linear_decode(A, A, None, A, 8, 896, 192, bf16, None) == _lib.SPK_EUNSUPPORTED
    assert lib.spk_linear_decode(A, A, A, A, 8, 896, 2048, bf16, None) == _lib.SPK_EUNSUPPORTED
    assert lib.spk_linear_decode(B, A, None, A, 8, 896, 896, bf16, None) == _lib.SPK_EINVAL
    assert b"aligned" in lib.spk_last_error()
    assert lib.spk_linear_decode(A, B, None, A, 8, 896, 4864, bf16, None) == _lib.SPK_EINVAL
    assert lib.spk_mlp_gate_pack(None, 20, 896, bf16, None, None) == _lib.SPK_EINVAL
    assert lib.spk_mlp_gate_lif(A, A, A, A, f32, A, 4, 8, 896, 4864, f16, None) == _lib.SPK_EUNSUPPORTED
    assert lib.spk_mlp_gate_lif(A, A, A, A, 7, A, 4, 8, 896, 4864, bf16, None) == _lib.SPK_EINVAL
    assert lib.spk_mlp_gate_lif(A, A, A, A, f32, A, 5, 8, 896, 4864, bf16, None) == _lib.SPK_EUNSUPPORTED
    assert lib.spk_mlp_gate_lif(A, A, A, A, f32, A, 4, 8, 256, 4864, bf16, None) == _lib.SPK_EUNSUPPORTED
    assert lib.spk_mlp_gate_lif(A, A, A, A, f32, A, 4, 8, 896, 512, bf16, None) == _lib.SPK_EUNSUPPORTED
    assert lib.spk_mlp_gate_lif(B, A, A, A, f32, A, 4, 8, 896, 4864, bf16, None) == _lib.SPK_EINVAL
    assert lib.spk_mlp_gate_packed_bytes(896, 4864) == 2 * 4864 * 896 * 2


def test_workspace_sizing():
    lib = _lib.load()
    # config 3 shape: one partition, no workspace
    assert lib.spk_decode_attn_workspace_bytes(4, 64, 14, 2, 64, 16, 12) == 0
    # config 4 shape: whole-sequence partitions, ordered longest first inside
    # the kernel, no workspace
    assert lib.spk_decode_attn_workspace_bytes(4, 256, 14, 2, 64, 16, 2048) == 0
    # past 4096 (sequence, partition) items a planner writes the launch order
    # (one int per work item + the item count)
    ws = lib.spk_decode_attn_workspace_bytes(1, 4100, 14, 2, 64, 16, 750)
    assert ws == (4100 * 1 * 2 + 1) * 4
    # a small batch is not split any further than a large one: partitions are
    # 32768 tokens whatever the batch (its sums do not depend on the batch)
    assert lib.spk_decode_attn_workspace_bytes(4, 8, 14, 2, 64, 16, 2048) == 0
    # past 32768 tokens: partial sums of 32768-token partitions (8 sequences,
    # 64k tokens: 2 partitions, 16 items, ordered inside the kernel)
    ws = lib.spk_decode_attn_workspace_bytes(4, 8, 14, 2, 64, 16, 4096)
    assert ws == 2 * 4 * 8 * 14 * 65 * 4
    # smaller blocks cap a partition at 2048 staged blocks (8-token blocks: 16384)
    ws = lib.spk_decode_attn_workspace_bytes(1, 1, 14, 2, 64, 8, 4096)
    assert ws == 2 * 1 * 1 * 14 * 65 * 4


def test_python_api_refuses_cpu_tensors():
    from spikeinfer_amd.kernels import lif_multistep, pack_spikes, paged_spike_attn_decode

    with pytest.raises(ValueError, match="GPU"):
        pack_spikes(torch.ones(2, 64))
    with pytest.raises(ValueError, match="GPU"):
        lif_multistep(torch.ones(4, 2, 64), torch.ones(64), torch.ones(64))
    q = torch.zeros(4, 1, 14, 2, dtype=torch.int32)
    kv = torch.zeros(4, 2, 32, 2, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU"):
        paged_spike_attn_decode(q, kv, kv, torch.zeros(1, 2, dtype=torch.int32),
                                torch.ones(1, dtype=torch.int32), 64, 16, 14, 2)
    with pytest.raises(ValueError, match="expected 1"):
        paged_spike_attn_decode(q, kv, kv, torch.zeros(1, 2, dtype=torch.int32),
                                torch.ones(1, dtype=torch.int32), 32, 16, 14, 2)


def test_sampler_workspace_size_and_validation():
    """The sliced sampler's workspace: per row, 8 slices of 256 candidates
    (x and index) plus a count, a maximum and a mass partial each; a short or
    misaligned one, or unknown stage bits, are refused before anything is
    launched."""
    lib = _lib.load()
    assert lib.spk_sample_workspace_bytes(64) == 64 * 8 * (2 * 256 * 4 + 16)
    assert lib.spk_sample_workspace_bytes(0) == 0
    args = lambda ws, nbytes, stages=3: (16, 2, 151936, 4, 151936, 16, None, None, None, None, None, None,
                                         None, 0, None, 0, None, 32, ws, nbytes, stages, None)
    assert lib.spk_sample_ws(*args(64, 100)) == _lib.SPK_EINVAL
    assert b"workspace" in lib.spk_last_error()
    assert lib.spk_sample_ws(*args(8, lib.spk_sample_workspace_bytes(4))) == _lib.SPK_EINVAL
    assert b"aligned" in lib.spk_last_error()
    assert lib.spk_sample_ws(*args(64, lib.spk_sample_workspace_bytes(4), 4)) == _lib.SPK_EINVAL
    assert b"stage" in lib.spk_last_error()


def test_sampler_stages_for_requests():
    """Which sliced sampler stages a batch of requests can use: greedy rows
    none, 0 < top_k <= 256 the top-k stage, every other top_k the open one
    when the row has a top-p or min-p cut."""
    from spikeinfer_amd.sampler import STAGE_OPEN, STAGE_TOPK, SamplingParams, stages_for

    assert stages_for([]) == 0
    assert stages_for([SamplingParams(temperature=0.0)]) == 0
    assert stages_for([SamplingParams(temperature=0.8, top_k=50)]) == STAGE_TOPK
    assert stages_for([SamplingParams(temperature=0.8, top_k=256)]) == STAGE_TOPK
    assert stages_for([SamplingParams(temperature=0.8, top_k=257, top_p=0.9)]) == STAGE_OPEN
    assert stages_for([SamplingParams(temperature=0.8, min_p=0.05)]) == STAGE_OPEN
    assert stages_for([SamplingParams(temperature=0.8)]) == 0  # a draw over the whole mass
    assert stages_for([SamplingParams(temperature=0.8, top_k=257)]) == 0
    assert stages_for([SamplingParams(top_p=0.9), SamplingParams(top_k=5)]) == STAGE_TOPK | STAGE_OPEN
    assert (STAGE_TOPK, STAGE_OPEN) == (1, 2)  # SPK_SAMPLE_STAGE_TOPK / _OPEN


def test_decode_gemms_decline_misaligned_outputs():
    """The fused MLP gate and linear_decode write y in 16-byte rows: a y off
    16 bytes is declined as unsupported (the caller then takes the library
    GEMM), a misaligned x or packed weight is an error; nothing is launched."""
    lib = _lib.load()
    args = lambda x, w, y: (x, w, 16, 16, _lib.SPK_F32, y, 4, 64, 896, 4864, _lib.SPK_BF16, None)
    assert lib.spk_mlp_gate_lif(*args(16, 16, 18)) == _lib.SPK_EUNSUPPORTED
    assert b"aligned" in lib.spk_last_error()
    assert lib.spk_mlp_gate_lif(*args(24, 16, 16)) == _lib.SPK_EINVAL
    # linear_decode, q/k/v shape (M 256, N 1152, K 896)
    assert lib.spk_linear_decode(16, 16, None, 18, 256, 1152, 896, _lib.SPK_BF16, None) == _lib.SPK_EUNSUPPORTED
    assert b"aligned" in lib.spk_last_error()


def test_combine_checks_the_partials_size():
    """spk_decode_attn_combine refuses a partials buffer smaller than
    num_parts * T*N*Hq*(head_dim+1) floats before launching anything."""
    lib = _lib.load()
    s4 = _i64(0, 0, 0, 1)
    need = 3 * 4 * 2 * 14 * 65 * 4
    rc = lib.spk_decode_attn_combine(16, need - 4, 3, 512, 16, 16, _lib.SPK_F32, s4, 4, 2, 14, 64, None)
    assert rc == _lib.SPK_EINVAL and b"partials buffer" in lib.spk_last_error()


def test_request_seeds_as_int64():
    """Request seeds are kept modulo 2**64 as two's-complement int64 (any seed
    torch.Generator.manual_seed takes, including 2**63 and above)."""
    from spikeinfer_amd.sampler import seed_as_int64

    assert seed_as_int64(0) == 0
    assert seed_as_int64(2 ** 63 - 1) == 2 ** 63 - 1
    assert seed_as_int64(2 ** 63) == -(2 ** 63)
    assert seed_as_int64(2 ** 64 - 1) == -1
    assert seed_as_int64(2 ** 64 + 5) == 5
    assert seed_as_int64(-1) == -1


def test_norm_gemms_validate_on_the_host():
    """The norm_* GEMM entry points refuse null inputs, misalignment and an
    h_out aliasing h before launching anything."""
    lib = _lib.load()
    bf16, f32 = _lib.SPK_BF16, _lib.SPK_F32
    A = 4096  # a 16-byte aligned stand-in address (never dereferenced)
    assert lib.spk_norm_linear_decode(None, A, A, A, 1e-6, A, None, A, 64, 1152, 896, bf16, None) == _lib.SPK_EINVAL
    assert lib.spk_norm_linear_decode(A, A + 16, A, A, 1e-6, A, None, A, 64, 1152, 896, bf16, None) == _lib.SPK_EINVAL
    assert b"alias" in lib.spk_last_error()
    assert lib.spk_norm_linear_decode(A, A + 16, A, A + 8, 1e-6, A, None, A, 64, 1152, 896, bf16, None) == _lib.SPK_EINVAL
    assert lib.spk_norm_linear_decode(A, A, A, None, 1e-6, A, None, A, 64, 1152, 1280, bf16, None) == _lib.SPK_EUNSUPPORTED
    assert lib.spk_norm_mlp_gate_lif(A, A + 16, A, A, 1e-6, A, A, A, f32, A, 4, 8, 896, 4864, bf16, None) == _lib.SPK_EINVAL
    assert lib.spk_norm_mlp_gate_lif(None, A, A, None, 1e-6, A, A, A, f32, A, 4, 8, 896, 4864, bf16, None) == _lib.SPK_EINVAL
