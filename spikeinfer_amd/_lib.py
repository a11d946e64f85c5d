"""ctypes binding of libspikeinfer_amd.so (the C ABI in include/spikeinfer_amd.h).

The library is loaded after ``torch`` so that its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already has in the process (same
SONAME): device pointers and streams from torch are then valid in the kernels.

Nothing here falls back to another implementation.  A missing library, or a
call on a non-GPU tensor, raises.
"""
from __future__ import annotations

import ctypes
import os
import struct

import torch

from .build import LIB_PATH

SPK_OK, SPK_EINVAL, SPK_EUNSUPPORTED, SPK_EHIP = 0, 1, 2, 3
SPK_F32, SPK_F16, SPK_BF16, SPK_U8, SPK_I32 = 0, 1, 2, 3, 4

_DTYPE_CODES = {
    torch.float32: SPK_F32,
    torch.float16: SPK_F16,
    torch.bfloat16: SPK_BF16,
    torch.uint8: SPK_U8,
    torch.bool: SPK_U8,
    torch.int32: SPK_I32,
}

ABI_VERSION = 3
DECODE_ATTN_SCRATCH_BYTES = 16 << 20  # SPK_DECODE_ATTN_SCRATCH_BYTES

_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_i32, _i64, _f32, _sz = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t

class SpkLifSite(ctypes.Structure):
    """struct SpkLifSite of include/spikeinfer_amd.h (one LIF-pack site)."""

    _fields_ = [
        ("x", _vp), ("x_strides", _i64 * 4), ("beta", _vp), ("threshold", _vp),
        ("param_dtype", _i32), ("scatter", _i32), ("out", _vp), ("out_strides", _i64 * 3),
        ("num_slots", _i64), ("n_tok", _i64), ("H", _i32), ("D", _i32),
    ]


_SITE_FORMAT = struct.Struct("<Q4qQQiiQ3qqqii")  # SpkLifSite, field by field (no padding)


def pack_lif_site(x, x_strides, beta, threshold, param_dtype, scatter, out, out_strides,
                  num_slots, n_tok, H, D) -> bytes:
    """The bytes of one SpkLifSite (struct.pack is ~10x cheaper per launch
    than building the ctypes Structure)."""
    return _SITE_FORMAT.pack(x, *x_strides, beta, threshold, param_dtype, scatter, out,
                             *out_strides, num_slots, n_tok, H, D)


# name -> (restype, argtypes); mirrors include/spikeinfer_amd.h
_SIGNATURES = {
    "spk_last_error": (ctypes.c_char_p, []),
    "spk_abi_version": (_i32, []),
    "spk_decode_attn": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _i64, _vp, _i64, _i64, _vp, _vp, _i32, _i64p,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp, _sz, _vp]),
    "spk_decode_attn_noalloc": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _i64, _vp, _i64, _i64, _vp, _vp, _i32, _i64p,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp]),
    "spk_decode_attn_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "spk_decode_attn_partials": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _i64, _vp, _i64, _i64, _vp, _i32, _i32, _i32, _i32,
        _i32, _i32, _i32, _f32, _i32, _vp, _sz, _vp]),
    "spk_decode_attn_combine": (_i32, [
        _vp, _sz, _i32, _i32, _vp, _vp, _i32, _i64p, _i32, _i32, _i32, _i32, _vp]),
    "spk_gather_unpack": (_i32, [
        _vp, _vp, _i64p, _i64, _vp, _i64, _i32, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp]),
    "spk_qkv_decode_attn": (_i32, [
        _vp, _i32, _i64p, _vp, _vp, _vp, _i64, _vp, _vp, _i32, _vp, _vp, _vp, _i64p, _i64, _vp,
        _i64, _i64, _vp, _vp, _i32, _i64p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp,
        _sz, _vp]),
    "spk_decode_scores": (_i32, [
        _vp, _i64p, _vp, _i64p, _i64, _vp, _i64, _i64, _vp, _vp, _i32, _i32, _i32, _i32,
        _i32, _i32, _i32, _vp]),
    "spk_lif_multistep": (_i32, [
        _vp, _i32, _i64p, _vp, _vp, _i32, _vp, _vp, _i32, _vp, _i32, _i64, _i32, _vp]),
    "spk_lif_pack_write": (_i32, [
        _vp, _i32, _i64p, _vp, _vp, _i32, _vp, _i64p, _vp, _i64, _vp, _i32, _i32, _i64,
        _i32, _i32, _vp]),
    "spk_lif_pack_write_sites": (_i32, [ctypes.c_char_p, _i32, _i32, _i32, _vp, _vp]),
    "spk_pack": (_i32, [_vp, _i32, _i64, _vp, _i64, _i32, _vp]),
    "spk_unpack": (_i32, [_vp, _i64, _i32, _vp, _i32, _vp]),
    "spk_add_rmsnorm": (_i32, [_vp, _vp, _vp, _vp, _i32, _i64, _i32, _f32, _vp]),
    "spk_rmsnorm_mean_t": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i64, _i32, _f32, _vp]),
    "spk_embed_rmsnorm": (_i32, [_vp, _vp, _i64, _vp, _vp, _vp, _i32, _i32, _i64, _i32, _f32, _vp]),
    "spk_qkv_rope_lif_pack": (_i32, [
        _vp, _i32, _i64p, _vp, _vp, _vp, _i64, _vp, _vp, _i32, _vp, _i64p, _i64, _vp, _vp, _i64p, _vp,
        _i64, _vp, _vp, _vp, _i32, _i64, _i32, _i32, _i32, _vp]),
    "spk_lif_gate_mul": (_i32, [_vp, _i32, _i64p, _vp, _vp, _i32, _vp, _i32, _i64, _i32, _vp]),
    "spk_mlp_gate_packed_bytes": (_sz, [_i32, _i32]),
    "spk_linear_pack": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp]),
    "spk_linear_decode": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    "spk_mlp_gate_pack": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp]),
    "spk_norm_linear_decode": (_i32, [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    "spk_norm_mlp_gate_lif": (_i32, [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32,
                                     _i32, _i32, _vp]),
    "spk_mlp_gate_lif": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _i32, _i32, _vp]),
    "spk_decode_advance": (_i32, [
        _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _i32, _vp, _vp,
        _vp]),
    "spk_sample": (_i32, [
        _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64,
        _vp, _vp, _vp]),
    "spk_sample_shared_bytes": (_sz, []),
    "spk_sample_workspace_bytes": (_sz, [_i32]),
    "spk_sample_ws": (_i32, [
        _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64,
        _vp, _vp, _vp, _sz, _i32, _vp]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lib = None


class KernelLibraryMissing(RuntimeError):
    """The HIP library is not built; run ``python -m spikeinfer_amd.build``."""


def load(path: str | None = None) -> ctypes.CDLL:
    """Loads (once) and returns the C-ABI library with typed signatures."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise KernelLibraryMissing(
            f"{path} not found: build it with `python -m spikeinfer_amd.build`"
        )
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.spk_abi_version() != ABI_VERSION:
        raise RuntimeError(
            f"{path} has ABI {lib.spk_abi_version()}, expected {ABI_VERSION}: rebuild it"
        )
    if path == LIB_PATH:
        _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Maps a C-ABI status to the exception the reference raises."""
    if rc == SPK_OK:
        return
    msg = load().spk_last_error().decode(errors="replace")
    if rc in (SPK_EINVAL, SPK_EUNSUPPORTED):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def strides(t: torch.Tensor, n: int | None = None):
    """Element strides of ``t`` as a ctypes int64 array (left-padded with 0)."""
    s = list(t.stride())
    if n is not None:
        s = [0] * (n - len(s)) + s
    return (ctypes.c_int64 * len(s))(*s)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one GPU; there is no CPU fallback in this package."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(
                "spikeinfer_amd kernels run on the GPU only; got a tensor on "
                f"{t.device} (the CPU implementation is test-only)"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev
