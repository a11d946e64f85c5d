"""LIF neuron on gfx950: dense spikes, and the fused LIF -> pack -> cache write.

Recurrence (spikeinfer/kernels/lif_triton.py:13-28, 96-105), per channel,
fp32 throughout, multiply and add rounded separately:

    r_t = H(U_{t-1} - theta)
    U_t = clamp(beta, 0, 1) * U_{t-1} + I_t - r_t * theta
    S_t = H(U_t - theta)
"""
from __future__ import annotations

import torch

from .. import _lib
from .packing import packed_width

_FLOATS = (torch.float32, torch.float16, torch.bfloat16)


def _param(p: torch.Tensor, n: int, dev) -> torch.Tensor:
    if p.device != dev:
        raise ValueError(f"LIF parameter on {p.device}, input on {dev}")
    p = p.reshape(n)
    if p.dtype not in _FLOATS:
        p = p.to(torch.float32)
    return p.contiguous()


def lif_multistep(x, beta, threshold, mem0=None, out_dtype=None, return_membrane=False):
    """Mirrors lif_multistep (lif_triton.py:141-233): ``[T, *mid, N]`` ->
    spikes of the same shape in ``out_dtype`` (default ``x.dtype``), plus the
    final fp32 membrane ``[*mid, N]`` when ``return_membrane``.

    Threshold > 0 is a precondition checked once by :func:`validate_thresholds`
    (a per-call check would need a device sync, illegal under graph capture).
    """
    assert x.ndim >= 2, "expected [T, *mid, N]"
    N = x.shape[-1]
    assert beta.numel() == N and threshold.numel() == N, (
        f"beta/threshold must match trailing dim: got {beta.numel()}/{threshold.numel()} vs N={N}"
    )
    dev = _lib.require_gpu(x)
    out_dtype = out_dtype or x.dtype
    if x.dtype not in _FLOATS:
        raise ValueError(f"lif_multistep input must be a float tensor, got {x.dtype}")
    orig_shape = x.shape
    T = orig_shape[0]
    x3 = x.reshape(T, -1, N)  # a view when the middle axes flatten, else a copy
    M = x3.shape[1]
    beta_c = _param(beta, N, dev)
    th_c = _param(threshold, N, dev)
    if beta_c.dtype != th_c.dtype:  # mixed dtypes: both to fp32 (exact), as the reference loads them
        beta_c, th_c = beta_c.float(), th_c.float()
    spike_dtype = torch.uint8 if out_dtype == torch.bool else out_dtype
    spikes = torch.empty((T, M, N), device=dev, dtype=spike_dtype)
    u_out = torch.empty((M, N), device=dev, dtype=torch.float32) if return_membrane else None
    u_in = None
    if mem0 is not None:
        u_in = mem0.reshape(M, N).to(device=dev, dtype=torch.float32).contiguous()
    _lib.check(
        _lib.load().spk_lif_multistep(
            x3.data_ptr(), _lib.dtype_code(x3.dtype), _lib.strides(x3),
            beta_c.data_ptr(), th_c.data_ptr(), _lib.dtype_code(beta_c.dtype),
            _lib.ptr(u_in), spikes.data_ptr(), _lib.dtype_code(spike_dtype),
            _lib.ptr(u_out), T, M, N, _lib.stream_of(dev),
        ),
        "lif_multistep",
    )
    if out_dtype == torch.bool:
        spikes = spikes.view(torch.bool)
    spikes = spikes.view(orig_shape)
    if return_membrane:
        return spikes, u_out.view(orig_shape[1:])
    return spikes


def lif_pack_write(
    x: torch.Tensor,
    beta: torch.Tensor,
    threshold: torch.Tensor,
    out: torch.Tensor,
    slot_mapping: torch.Tensor | None = None,
    spikes_out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Fused LIF + bit-pack (+ paged-cache scatter) for one q/k/v site.

    Replaces ``pack_spikes(lif_multistep(x, ...))`` followed, for k and v, by
    ``cache.index_copy_(2, slot_mapping, ...)`` (modeling_fast.py:132-134,
    attention.py:138-139, :146-149).

    Args:
        x: ``[T, n_tok, H, D]`` input current, any strides (e.g. the projection
            output viewed per head, no copy).
        beta, threshold: ``[D]``.
        out: with ``slot_mapping`` None, the packed buffer ``int32 [T, n_tok,
            H, W]``; otherwise the paged cache ``int32 [T, H, num_slots, W]``
            that token ``i`` is scattered into at ``slot_mapping[i]`` (int64;
            slots outside the cache are skipped).
        spikes_out: optional dense ``[T, n_tok, H, D]`` contiguous 0/1 output.

    Returns ``out``.
    """
    if x.ndim != 4:
        raise ValueError(f"expected x as [T, n_tok, H, D], got shape {tuple(x.shape)}")
    T, n_tok, H, D = x.shape
    dev = _lib.require_gpu(x, out, slot_mapping, spikes_out)
    if x.dtype not in _FLOATS:
        raise ValueError(f"lif_pack_write input must be a float tensor, got {x.dtype}")
    W = packed_width(D)
    if out.dtype != torch.int32 or out.ndim != 4 or out.shape[-1] != W or out.stride(-1) != 1:
        raise ValueError(f"packed output must be int32 [..., {W}] with a contiguous word axis")
    if slot_mapping is None:
        if tuple(out.shape[:3]) != (T, n_tok, H):
            raise ValueError(f"packed buffer shape {tuple(out.shape)} != {(T, n_tok, H, W)}")
        pstr = (out.stride(0), out.stride(1), out.stride(2))
        num_slots, slots_ptr = 0, None
    else:
        if out.shape[0] != T or out.shape[1] != H:
            raise ValueError(f"cache shape {tuple(out.shape)} does not match T={T}, H={H}")
        if slot_mapping.numel() < n_tok:
            raise ValueError(f"slot_mapping has {slot_mapping.numel()} entries for {n_tok} tokens")
        if slot_mapping.dtype != torch.int64:
            slot_mapping = slot_mapping.to(torch.int64)
        slot_mapping = slot_mapping.contiguous()
        pstr = (out.stride(0), out.stride(1), out.stride(2))
        num_slots, slots_ptr = out.shape[2], slot_mapping.data_ptr()
    spike_dtype = 0
    if spikes_out is not None:
        if tuple(spikes_out.shape) != (T, n_tok, H, D) or not spikes_out.is_contiguous():
            raise ValueError("spikes_out must be a contiguous [T, n_tok, H, D] tensor")
        sd = torch.uint8 if spikes_out.dtype == torch.bool else spikes_out.dtype
        spike_dtype = _lib.dtype_code(sd)
    beta_c = _param(beta, D, dev)
    th_c = _param(threshold, D, dev)
    if beta_c.dtype != th_c.dtype:  # mixed dtypes: both to fp32 (exact), as the reference loads them
        beta_c, th_c = beta_c.float(), th_c.float()
    _lib.check(
        _lib.load().spk_lif_pack_write(
            x.data_ptr(), _lib.dtype_code(x.dtype), _lib.strides(x),
            beta_c.data_ptr(), th_c.data_ptr(), _lib.dtype_code(beta_c.dtype),
            out.data_ptr(), (_lib.ctypes.c_int64 * 3)(*pstr), slots_ptr, num_slots,
            _lib.ptr(spikes_out), spike_dtype, T, n_tok, H, D, _lib.stream_of(dev),
        ),
        "lif_pack_write",
    )
    return out


def validate_thresholds(model):
    """Checks ``threshold > 0`` at every LIF site (lif_triton.py:236-253).

    Call once after loading weights: it synchronises the device.
    """
    bad = []
    for name, module in model.named_modules():
        lif = getattr(module, "lif", None)
        th = getattr(lif, "threshold", None) if lif is not None else None
        if th is None:
            th = getattr(module, "lif_threshold", None)
        if th is not None and not bool(torch.all(th > 0)):
            bad.append(f"{name} (min={th.min().item():.4g})")
    if bad:
        raise ValueError(
            "lif_multistep requires threshold > 0; violated at: " + ", ".join(bad)
        )
    return True
