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
    if p.dtype in _FLOATS and p.dim() == 1 and p.shape[0] == n and p.is_contiguous() and p.device == dev:
        return p  # the usual case, without the reshape/copy calls (host time per launch)
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
    if slot_mapping is not None:
        if slot_mapping.dtype != torch.int64:
            slot_mapping = slot_mapping.to(torch.int64)
        slot_mapping = slot_mapping.contiguous()
    if spikes_out is not None:
        site = _site(x, beta, threshold, out, slot_mapping)
        T, n_tok, H, D = x.shape
        if tuple(spikes_out.shape) != (T, n_tok, H, D) or not spikes_out.is_contiguous():
            raise ValueError("spikes_out must be a contiguous [T, n_tok, H, D] tensor")
        _lib.require_gpu(spikes_out)
        sd = torch.uint8 if spikes_out.dtype == torch.bool else spikes_out.dtype
        st = _lib.SpkLifSite.from_buffer_copy(site["struct"])
        _lib.check(
            _lib.load().spk_lif_pack_write(
                x.data_ptr(), _lib.dtype_code(x.dtype), st.x_strides, st.beta, st.threshold,
                st.param_dtype, out.data_ptr(), st.out_strides, _lib.ptr(site["slots"]),
                st.num_slots, spikes_out.data_ptr(), _lib.dtype_code(sd), T, n_tok, H, D,
                _lib.stream_of(x.device),
            ),
            "lif_pack_write",
        )
        return out
    lif_pack_write_sites([(x, beta, threshold, out, slot_mapping is not None)], slot_mapping)
    return out


def _site(x, beta, threshold, out, slot_mapping):
    """Validates one LIF-pack site and returns its SpkLifSite (plus the
    tensors it points into, kept alive by the caller until the launch)."""
    if x.ndim != 4:
        raise ValueError(f"expected x as [T, n_tok, H, D], got shape {tuple(x.shape)}")
    T, n_tok, H, D = x.shape
    dev = _lib.require_gpu(x, out, slot_mapping)
    if x.dtype not in _FLOATS:
        raise ValueError(f"lif_pack_write input must be a float tensor, got {x.dtype}")
    W = packed_width(D)
    if out.dtype != torch.int32 or out.ndim != 4 or out.shape[-1] != W or out.stride(-1) != 1:
        raise ValueError(f"packed output must be int32 [..., {W}] with a contiguous word axis")
    if slot_mapping is None:
        if tuple(out.shape[:3]) != (T, n_tok, H):
            raise ValueError(f"packed buffer shape {tuple(out.shape)} != {(T, n_tok, H, W)}")
        num_slots = 0
    else:
        if out.shape[0] != T or out.shape[1] != H:
            raise ValueError(f"cache shape {tuple(out.shape)} does not match T={T}, H={H}")
        if slot_mapping.numel() < n_tok:
            raise ValueError(f"slot_mapping has {slot_mapping.numel()} entries for {n_tok} tokens")
        num_slots = out.shape[2]
    beta_c = _param(beta, D, dev)
    th_c = _param(threshold, D, dev)
    if beta_c.dtype != th_c.dtype:  # mixed dtypes: both to fp32 (exact), as the reference loads them
        beta_c, th_c = beta_c.float(), th_c.float()
    os_ = out.stride()
    st = _lib.pack_lif_site(x.data_ptr(), x.stride(), beta_c.data_ptr(), th_c.data_ptr(),
                            _lib.dtype_code(beta_c.dtype), 0 if slot_mapping is None else 1,
                            out.data_ptr(), os_[:3], num_slots, n_tok, H, D)
    return {"struct": st, "keep": (beta_c, th_c), "slots": slot_mapping, "T": T, "dev": dev}


def lif_pack_write_sites(sites, slot_mapping: torch.Tensor | None = None) -> None:
    """Several :func:`lif_pack_write` sites in one launch (1 to 4), e.g. an
    attention layer's k and v (scattered into their caches by
    ``slot_mapping``) and its decode queries (into the packed buffer).

    Args:
        sites: sequence of ``(x, beta, threshold, out, scatter)``; ``scatter``
            True sends token ``i`` to cache slot ``slot_mapping[i]`` (the cache
            form of ``out``), False writes the packed buffer form.  All ``x``
            share one dtype and T.
        slot_mapping: int64 ``[n_tok]``, needed when any site scatters.

    Same bits as one :func:`lif_pack_write` per site; replaces the three LIF
    sites of attention.py:138-149 / modeling_fast.py:132-134.
    """
    sites = list(sites)
    if not 1 <= len(sites) <= 4:
        raise ValueError(f"lif_pack_write_sites takes 1 to 4 sites, got {len(sites)}")
    if slot_mapping is not None:
        if slot_mapping.dtype != torch.int64:
            slot_mapping = slot_mapping.to(torch.int64)
        slot_mapping = slot_mapping.contiguous()
    built = []
    for x, beta, th, out, scatter in sites:
        if scatter and slot_mapping is None:
            raise ValueError("a scattering site needs slot_mapping")
        built.append(_site(x, beta, th, out, slot_mapping if scatter else None))
    x_dtype = sites[0][0].dtype
    T = built[0]["T"]
    dev = built[0]["dev"]
    for (x, *_), b in zip(sites, built):
        if x.dtype != x_dtype or b["T"] != T or b["dev"] != dev:
            raise ValueError("lif_pack_write_sites: every site needs the same x dtype, T and device")
    arr = b"".join(b["struct"] for b in built)
    _lib.check(
        _lib.load().spk_lif_pack_write_sites(
            arr, len(built), _lib.dtype_code(x_dtype), T, _lib.ptr(slot_mapping),
            _lib.stream_of(dev)),
        "lif_pack_write_sites",
    )


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
