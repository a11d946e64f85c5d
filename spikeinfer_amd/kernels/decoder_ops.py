"""Decoder-step operators around the GEMMs (HIP, through the C-ABI).

Each replaces a torch composition of the reference's layer-major forward
(spikeinfer/modeling_fast.py) with one launch; shapes follow that forward's
flattened, paged form ``[T, n_tok, ...]``.
"""
from __future__ import annotations

import math

import torch

from .. import _lib

_VEC_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _contig_rows(t: torch.Tensor, name: str) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def add_rmsnorm(h: torch.Tensor, delta: torch.Tensor | None, weight: torch.Tensor,
                eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """``h += delta`` (in place, rounded to h's dtype), then Qwen2RMSNorm(h).

    ``h``/``delta``/``out`` ``[..., hidden]`` contiguous, ``weight [hidden]``.
    Returns ``out`` (allocated like ``h`` when None).
    """
    dev = _lib.require_gpu(h, delta, weight, out)
    if h.dtype not in _VEC_DTYPES:
        raise ValueError(f"add_rmsnorm: unsupported dtype {h.dtype}")
    for name, t in (("h", h), ("delta", delta), ("weight", weight), ("out", out)):
        if t is not None:
            _contig_rows(t, name)
            if t.dtype != h.dtype:
                raise ValueError(f"add_rmsnorm: {name} is {t.dtype}, h is {h.dtype}")
    if delta is not None and delta.shape != h.shape:
        raise ValueError(f"add_rmsnorm: delta {tuple(delta.shape)} vs h {tuple(h.shape)}")
    hidden = h.shape[-1]
    if weight.numel() != hidden:
        raise ValueError(f"add_rmsnorm: weight has {weight.numel()} entries, hidden is {hidden}")
    if out is None:
        out = torch.empty_like(h)
    _lib.check(
        _lib.load().spk_add_rmsnorm(
            h.data_ptr(), _lib.ptr(delta), weight.data_ptr(), out.data_ptr(),
            _lib.dtype_code(h.dtype), h.numel() // hidden, hidden, float(eps), _lib.stream_of(dev),
        ),
        "add_rmsnorm",
    )
    return out


def embed_rmsnorm(ids: torch.Tensor, embed: torch.Tensor, weight: torch.Tensor, eps: float,
                  T: int, h: torch.Tensor | None = None,
                  out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Embedding rows of ``ids`` broadcast over ``T`` steps, and their RMSNorm.

    Returns ``(h, x)``, both ``[T, n, hidden]``: ``h[t] = embed[ids]`` and
    ``x[t] = Qwen2RMSNorm(h[t])``.
    """
    dev = _lib.require_gpu(ids, embed, weight, h, out)
    if ids.dtype != torch.int64 or ids.ndim != 1 or not ids.is_contiguous():
        raise ValueError("embed_rmsnorm: ids must be a contiguous int64 vector")
    if embed.ndim != 2 or not embed.is_contiguous() or embed.dtype not in _VEC_DTYPES:
        raise ValueError("embed_rmsnorm: embed must be a contiguous [vocab, hidden] float matrix")
    vocab, hidden = embed.shape
    if weight.numel() != hidden or weight.dtype != embed.dtype or not weight.is_contiguous():
        raise ValueError(f"embed_rmsnorm: weight must be {hidden} contiguous {embed.dtype} entries")
    n = ids.numel()
    shape = (T, n, hidden)
    h = torch.empty(shape, dtype=embed.dtype, device=dev) if h is None else h
    out = torch.empty(shape, dtype=embed.dtype, device=dev) if out is None else out
    for name, t in (("h", h), ("out", out)):
        if tuple(t.shape) != shape or t.dtype != embed.dtype or not t.is_contiguous():
            raise ValueError(f"embed_rmsnorm: {name} must be contiguous {shape} {embed.dtype}")
    _lib.check(
        _lib.load().spk_embed_rmsnorm(
            ids.data_ptr(), embed.data_ptr(), vocab, weight.data_ptr(), h.data_ptr(), out.data_ptr(),
            _lib.dtype_code(embed.dtype), T, n, hidden, float(eps), _lib.stream_of(dev),
        ),
        "embed_rmsnorm",
    )
    return h, out


def rmsnorm_mean_t(h: torch.Tensor, weight: torch.Tensor, eps: float,
                   out: torch.Tensor | None = None, delta: torch.Tensor | None = None) -> torch.Tensor:
    """``RMSNorm(h + delta).mean(dim=0)`` for ``h [T, rows, hidden]``
    contiguous (``delta`` optional, same shape; h is not modified)."""
    dev = _lib.require_gpu(h, weight, out, delta)
    if h.ndim != 3:
        raise ValueError("rmsnorm_mean_t: expected h as [T, rows, hidden]")
    _contig_rows(h, "h")
    if delta is not None:
        _contig_rows(delta, "delta")
        if delta.shape != h.shape or delta.dtype != h.dtype:
            raise ValueError("rmsnorm_mean_t: delta must match h")
    T, rows, hidden = h.shape
    if out is None:
        out = torch.empty((rows, hidden), dtype=h.dtype, device=dev)
    _lib.check(
        _lib.load().spk_rmsnorm_mean_t(
            h.data_ptr(), _lib.ptr(delta), weight.data_ptr(), out.data_ptr(), _lib.dtype_code(h.dtype), T, rows,
            hidden, float(eps), _lib.stream_of(dev),
        ),
        "rmsnorm_mean_t",
    )
    return out


def qkv_rope_lif_pack(
    qkv: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    beta: torch.Tensor,
    threshold: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    q_packed: torch.Tensor | None = None,
    n_q: int = 0,
    dense: tuple[torch.Tensor | None, torch.Tensor | None, torch.Tensor | None] | None = None,
    positions: torch.Tensor | None = None,
) -> torch.Tensor | None:
    """RoPE -> LIF -> pack for the q/k/v site of one layer.

    Args:
        qkv: ``[T, n_tok, (Hq + 2 Hkv) * D]`` concatenated projection output
            (channel stride 1).
        cos, sin: ``[n_tok, D]`` rotary tables in qkv's dtype, or, with
            ``positions`` (int64 ``[n_tok]``), ``[rows, D]`` tables indexed by
            each token's position.
        beta, threshold: ``[3, D]`` (q, k, v sites).
        k_cache, v_cache: the layer's ``int32 [T, Hkv, slots, W]`` caches;
            token ``i`` is written at ``slot_mapping[i]``.
        q_packed: ``int32 [T, n_q, Hq, W]`` receiving tokens ``[0, n_q)``.
        dense: optional ``[T, H, n_tok, D]`` outputs of the 0/1 spikes per site.
    Returns ``q_packed``.
    """
    dev = _lib.require_gpu(qkv, cos, sin, beta, threshold, k_cache, v_cache, slot_mapping, q_packed,
                           positions)
    if qkv.ndim != 3 or qkv.stride(-1) != 1:
        raise ValueError("qkv must be [T, n_tok, C] with a contiguous channel axis")
    T, n_tok, C = qkv.shape
    if C != (num_q_heads + 2 * num_kv_heads) * head_dim:
        raise ValueError(f"qkv has {C} channels, expected {(num_q_heads + 2 * num_kv_heads) * head_dim}")
    rows = cos.shape[0] if positions is not None else n_tok
    if positions is not None:
        if positions.dtype != torch.int64 or not positions.is_contiguous() or positions.numel() < n_tok:
            raise ValueError(f"positions must be a contiguous int64 vector of >= {n_tok} entries")
        if rows < 1:
            raise ValueError("rotary tables need at least one row")
    for name, t in (("cos", cos), ("sin", sin)):
        if t.ndim != 2 or tuple(t.shape) != (rows, head_dim) or not t.is_contiguous() or t.dtype != qkv.dtype:
            raise ValueError(f"{name} must be a contiguous [{rows}, {head_dim}] {qkv.dtype} tensor")
    beta = beta.reshape(3, head_dim).contiguous()
    threshold = threshold.reshape(3, head_dim).to(beta.dtype).contiguous()
    if slot_mapping.dtype != torch.int64:
        slot_mapping = slot_mapping.to(torch.int64)
    slot_mapping = slot_mapping.contiguous()
    if slot_mapping.numel() < n_tok:
        raise ValueError(f"slot_mapping has {slot_mapping.numel()} entries for {n_tok} tokens")
    qs = _lib.strides(q_packed) if q_packed is not None else (_lib.ctypes.c_int64 * 3)(0, 0, 0)
    if q_packed is not None:
        if q_packed.dtype != torch.int32 or q_packed.ndim != 4 or q_packed.shape[0] != T \
                or q_packed.shape[1] < n_q or q_packed.shape[2] != num_q_heads:
            raise ValueError(f"q_packed must be int32 [T, >= {n_q}, {num_q_heads}, W]")
        qs = (_lib.ctypes.c_int64 * 3)(*q_packed.stride()[:3])
    elif n_q:
        raise ValueError("n_q > 0 needs q_packed")
    dq, dk, dv = dense if dense is not None else (None, None, None)
    for t, H in ((dq, num_q_heads), (dk, num_kv_heads), (dv, num_kv_heads)):
        if t is not None and (tuple(t.shape) != (T, H, n_tok, head_dim) or not t.is_contiguous()
                              or t.dtype != qkv.dtype):
            raise ValueError(f"dense spikes must be contiguous [T, {H}, {n_tok}, {head_dim}] {qkv.dtype}")
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("k and v caches must have the same shape and strides")
    _lib.check(
        _lib.load().spk_qkv_rope_lif_pack(
            qkv.data_ptr(), _lib.dtype_code(qkv.dtype), (_lib.ctypes.c_int64 * 2)(*qkv.stride()[:2]),
            cos.data_ptr(), sin.data_ptr(), _lib.ptr(positions), rows if positions is not None else 0,
            beta.data_ptr(), threshold.data_ptr(),
            _lib.dtype_code(beta.dtype), _lib.ptr(q_packed), qs, n_q,
            k_cache.data_ptr(), v_cache.data_ptr(), (_lib.ctypes.c_int64 * 3)(*k_cache.stride()[:3]),
            slot_mapping.data_ptr(), k_cache.shape[2], _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv),
            T, n_tok, num_q_heads, num_kv_heads, head_dim, _lib.stream_of(dev),
        ),
        "qkv_rope_lif_pack",
    )
    return q_packed


def qkv_decode_attention(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                         positions: torch.Tensor, beta: torch.Tensor, threshold: torch.Tensor,
                         k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                         block_tables: torch.Tensor, seq_lens: torch.Tensor, num_q_heads: int,
                         num_kv_heads: int, block_size: int, out: torch.Tensor,
                         workspace: torch.Tensor | None = None) -> bool:
    """Fused decode step of one layer's attention: the q/k/v spikes of the
    ``N = qkv.shape[1]`` decode tokens (as :func:`qkv_rope_lif_pack`), their
    k/v words into the cache, and attention into ``out [T, N, Hq, 64]``.

    Returns False, having done nothing, when the shape is outside the fused
    kernel (head_dim 64, Hq/Hkv <= 8, T <= 8); the caller then runs the two
    separate operations.
    """
    from .spike_attention import decode_attn_workspace_bytes

    dev = _lib.require_gpu(qkv, cos, sin, positions, beta, threshold, k_cache, v_cache, slot_mapping,
                           block_tables, seq_lens, out, workspace)
    T, n, C = qkv.shape
    D = 64
    if (C != (num_q_heads + 2 * num_kv_heads) * D or num_q_heads % num_kv_heads
            or num_q_heads // num_kv_heads > 8 or T > 8 or k_cache.shape[-1] != 2):
        return False
    if qkv.stride(-1) != 1 or positions.dtype != torch.int64 or not positions.is_contiguous():
        raise ValueError("qkv needs a contiguous channel axis and positions contiguous int64")
    if (positions.numel() < n or slot_mapping.numel() < n or seq_lens.numel() < n
            or block_tables.ndim != 2 or block_tables.shape[0] < n):
        raise ValueError(f"positions, slot_mapping, seq_lens and block_tables need {n} rows")
    for name, t in (("cos", cos), ("sin", sin)):
        if t.ndim != 2 or t.shape[1] != D or not t.is_contiguous() or t.dtype != qkv.dtype:
            raise ValueError(f"{name} must be a contiguous [rows, {D}] {qkv.dtype} table")
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("k and v caches must have the same shape and strides")
    if tuple(out.shape) != (T, n, num_q_heads, D):
        raise ValueError(f"out must be [{T}, {n}, {num_q_heads}, {D}]")
    # the fused kernel reads fp32 parameters: the upcast is exact (bf16/f16 -> fp32),
    # and a model that keeps them in fp32 (SpikingDecoder does) pays no copy here
    beta = beta.reshape(3, D).float().contiguous()
    threshold = threshold.reshape(3, D).float().contiguous()
    slot_mapping = slot_mapping.to(torch.int64).contiguous()
    block_tables = block_tables.to(torch.int32)
    seq_lens = seq_lens.to(torch.int32).contiguous()
    max_blocks = block_tables.shape[1]
    need = decode_attn_workspace_bytes(T, n, num_q_heads, num_kv_heads, D, block_size, max_blocks)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    rc = _lib.load().spk_qkv_decode_attn(
        qkv.data_ptr(), _lib.dtype_code(qkv.dtype), (_lib.ctypes.c_int64 * 2)(*qkv.stride()[:2]),
        cos.data_ptr(), sin.data_ptr(), positions.data_ptr(), cos.shape[0], beta.data_ptr(),
        threshold.data_ptr(), _lib.dtype_code(beta.dtype), slot_mapping.data_ptr(),
        k_cache.data_ptr(), v_cache.data_ptr(), _lib.strides(k_cache), k_cache.shape[2],
        block_tables.data_ptr(), block_tables.stride(0), block_tables.stride(1), seq_lens.data_ptr(),
        out.data_ptr(), _lib.dtype_code(out.dtype), _lib.strides(out), T, n, num_q_heads,
        num_kv_heads, D, block_size, max_blocks, 1.0 / math.sqrt(D),
        _lib.ptr(workspace) if need else None, need, _lib.stream_of(dev))
    if rc == _lib.SPK_EUNSUPPORTED:
        return False
    _lib.check(rc, "qkv_decode_attention")
    return True


def lif_gate_mul(gate_up: torch.Tensor, beta: torch.Tensor, threshold: torch.Tensor,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """``LIF(gate) * up`` for ``gate_up [T, rows, 2I]`` (gate columns first).

    Returns ``[T, rows, I]`` contiguous in gate_up's dtype.
    """
    dev = _lib.require_gpu(gate_up, beta, threshold, out)
    if gate_up.ndim != 3 or gate_up.stride(-1) != 1:
        raise ValueError("gate_up must be [T, rows, 2I] with a contiguous channel axis")
    T, rows, I2 = gate_up.shape
    I = I2 // 2
    if I2 % 2 or beta.numel() != I or threshold.numel() != I:
        raise ValueError(f"gate_up has {I2} channels; beta/threshold need {I} entries")
    if out is None:
        out = torch.empty((T, rows, I), dtype=gate_up.dtype, device=dev)
    elif tuple(out.shape) != (T, rows, I) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{T}, {rows}, {I}]")
    beta = beta.contiguous()
    threshold = threshold.to(beta.dtype).contiguous()
    _lib.check(
        _lib.load().spk_lif_gate_mul(
            gate_up.data_ptr(), _lib.dtype_code(gate_up.dtype),
            (_lib.ctypes.c_int64 * 2)(*gate_up.stride()[:2]), beta.data_ptr(), threshold.data_ptr(),
            _lib.dtype_code(beta.dtype), out.data_ptr(), T, rows, I, _lib.stream_of(dev),
        ),
        "lif_gate_mul",
    )
    return out


def pack_gate_up(w_gu: torch.Tensor) -> torch.Tensor:
    """Reorders the concatenated gate|up weight ``[2I, hidden]`` (bf16) into the
    operand order of :func:`mlp_gate_lif`; done once per weight."""
    dev = _lib.require_gpu(w_gu)
    if w_gu.ndim != 2 or w_gu.dtype != torch.bfloat16 or not w_gu.is_contiguous():
        raise ValueError("w_gu must be a contiguous bf16 [2I, hidden] tensor")
    I2, hidden = w_gu.shape
    if I2 % 32 or hidden % 32:
        raise ValueError(f"w_gu shape {tuple(w_gu.shape)}: 2I must be a multiple of 32, hidden of 32")
    lib = _lib.load()
    out = torch.empty(lib.spk_mlp_gate_packed_bytes(hidden, I2 // 2) // 2, dtype=torch.bfloat16,
                      device=dev)
    _lib.check(lib.spk_mlp_gate_pack(w_gu.data_ptr(), I2 // 2, hidden, _lib.dtype_code(w_gu.dtype),
                                     out.data_ptr(), _lib.stream_of(dev)), "mlp_gate_pack")
    return out


def pack_linear(w: torch.Tensor) -> torch.Tensor:
    """Reorders a bf16 weight ``[N, K]`` into the operand order of
    :func:`linear_decode`; done once per weight."""
    dev = _lib.require_gpu(w)
    if w.ndim != 2 or w.dtype != torch.bfloat16 or not w.is_contiguous():
        raise ValueError("w must be a contiguous bf16 [N, K] tensor")
    N, K = w.shape
    if N % 16 or K % 32:
        raise ValueError(f"w shape {tuple(w.shape)}: N must be a multiple of 16, K of 32")
    out = torch.empty_like(w)
    _lib.check(_lib.load().spk_linear_pack(w.data_ptr(), N, K, _lib.dtype_code(w.dtype), out.data_ptr(),
                                           _lib.stream_of(dev)), "linear_pack")
    return out


def linear_decode(x: torch.Tensor, w_packed: torch.Tensor, bias: torch.Tensor | None = None,
                  out: torch.Tensor | None = None) -> torch.Tensor | None:
    """``x @ W^T (+ bias)`` for a decode-sized ``x [..., K]`` (at most 256 rows)
    from :func:`pack_linear`'s weight, into ``out`` when given (contiguous);
    None when the shape is outside the kernel's range (the caller then uses
    ``F.linear``)."""
    dev = _lib.require_gpu(x, w_packed, bias, out)
    if x.dtype != torch.bfloat16 or w_packed.ndim != 2 or w_packed.shape[1] != x.shape[-1]:
        raise ValueError("x must be bf16 [..., K] and w_packed [N, K]")
    N, K = w_packed.shape
    if bias is not None and (bias.numel() != N or bias.dtype != torch.bfloat16):
        raise ValueError(f"bias must be bf16 with {N} entries")
    x2 = x.reshape(-1, K).contiguous()
    if out is None:
        y = torch.empty((x2.shape[0], N), dtype=x.dtype, device=dev)
    elif out.shape[-1] != N or out.numel() != x2.shape[0] * N or not out.is_contiguous() \
            or out.dtype != x.dtype:
        raise ValueError(f"out must be a contiguous {x.dtype} tensor of {x2.shape[0]} x {N}")
    else:
        y = out
    rc = _lib.load().spk_linear_decode(
        x2.data_ptr(), w_packed.data_ptr(), bias.contiguous().data_ptr() if bias is not None else None,
        y.data_ptr(), x2.shape[0], N, K, _lib.dtype_code(x.dtype), _lib.stream_of(dev))
    if rc == _lib.SPK_EUNSUPPORTED:
        return None
    _lib.check(rc, "linear_decode")
    return y if out is not None else y.view(*x.shape[:-1], N)


def mlp_gate_lif(x: torch.Tensor, w_packed: torch.Tensor, beta: torch.Tensor,
                 threshold: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor | None:
    """``LIF(x @ W_g^T) * (x @ W_u^T)`` for ``x [T, n_tok, hidden]`` in one
    launch (modeling_fast.py:186-190), from :func:`pack_gate_up`'s weight.

    Returns ``[T, n_tok, I]``, or None when the shape is outside the kernel's
    range (the caller then runs the GEMM and :func:`lif_gate_mul`).
    """
    dev = _lib.require_gpu(x, w_packed, beta, threshold, out)
    if x.ndim != 3 or x.dtype != torch.bfloat16:
        raise ValueError("x must be a bf16 [T, n_tok, hidden] tensor")
    T, n, hidden = x.shape
    I = beta.numel()
    if threshold.numel() != I or w_packed.numel() * w_packed.element_size() != 4 * I * hidden:
        raise ValueError(f"packed weight / beta / threshold do not match hidden={hidden}, I={I}")
    x = x.contiguous()
    if out is None:
        out = torch.empty((T, n, I), dtype=x.dtype, device=dev)
    elif tuple(out.shape) != (T, n, I) or not out.is_contiguous() or out.dtype != x.dtype:
        raise ValueError(f"out must be contiguous bf16 [{T}, {n}, {I}]")
    # fp32 parameters (exact upcast; SpikingDecoder keeps them in fp32, so no copy)
    beta = beta.float().contiguous()
    threshold = threshold.float().contiguous()
    rc = _lib.load().spk_mlp_gate_lif(
        x.data_ptr(), w_packed.data_ptr(), beta.data_ptr(), threshold.data_ptr(),
        _lib.dtype_code(beta.dtype), out.data_ptr(), T, n, hidden, I, _lib.dtype_code(x.dtype),
        _lib.stream_of(dev))
    if rc == _lib.SPK_EUNSUPPORTED:
        return None
    _lib.check(rc, "mlp_gate_lif")
    return out


def _norm_inputs(h, delta, norm_weight, h_out, name):
    """Checks of the residual-stream inputs of the norm_* GEMMs."""
    if h.dtype != torch.bfloat16 or delta.dtype != h.dtype or norm_weight.dtype != h.dtype:
        raise ValueError(f"{name}: h, delta and norm_weight must be bf16")
    if delta.shape != h.shape or not h.is_contiguous() or not delta.is_contiguous():
        raise ValueError(f"{name}: h and delta must be contiguous tensors of one shape")
    if norm_weight.numel() != h.shape[-1] or not norm_weight.is_contiguous():
        raise ValueError(f"{name}: norm_weight must be contiguous with hidden={h.shape[-1]} entries")
    if h_out is not None and (h_out.shape != h.shape or h_out.dtype != h.dtype or not h_out.is_contiguous()):
        raise ValueError(f"{name}: h_out must be a contiguous bf16 tensor shaped like h")


def norm_linear_decode(h: torch.Tensor, delta: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                       w_packed: torch.Tensor, bias: torch.Tensor | None = None,
                       out: torch.Tensor | None = None,
                       h_out: torch.Tensor | None = None) -> torch.Tensor | None:
    """``linear_decode(add_rmsnorm(h, delta, norm_weight), w_packed, bias)`` in
    one launch, without changing ``h``: ``h_out`` (when given) receives ``h +
    delta``.  ``h``/``delta`` ``[..., K]`` bf16.  Identical values to the two
    launches; None when the shape is outside the kernel's range."""
    dev = _lib.require_gpu(h, delta, norm_weight, w_packed, bias, out, h_out)
    _norm_inputs(h, delta, norm_weight, h_out, "norm_linear_decode")
    N, K = w_packed.shape
    if h.shape[-1] != K:
        raise ValueError(f"norm_linear_decode: h has {h.shape[-1]} columns, the weight {K}")
    if bias is not None and (bias.numel() != N or bias.dtype != torch.bfloat16):
        raise ValueError(f"bias must be bf16 with {N} entries")
    M = h.numel() // K
    if out is None:
        out = torch.empty((*h.shape[:-1], N), dtype=h.dtype, device=dev)
    elif out.numel() != M * N or not out.is_contiguous() or out.dtype != h.dtype:
        raise ValueError(f"out must be a contiguous bf16 tensor of {M} x {N}")
    rc = _lib.load().spk_norm_linear_decode(
        h.data_ptr(), delta.data_ptr(), norm_weight.data_ptr(), _lib.ptr(h_out), float(eps),
        w_packed.data_ptr(), bias.contiguous().data_ptr() if bias is not None else None, out.data_ptr(),
        M, N, K, _lib.dtype_code(h.dtype), _lib.stream_of(dev))
    if rc == _lib.SPK_EUNSUPPORTED:
        return None
    _lib.check(rc, "norm_linear_decode")
    return out


def norm_mlp_gate_lif(h: torch.Tensor, delta: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                      w_packed: torch.Tensor, beta: torch.Tensor, threshold: torch.Tensor,
                      out: torch.Tensor | None = None,
                      h_out: torch.Tensor | None = None) -> torch.Tensor | None:
    """``mlp_gate_lif(add_rmsnorm(h, delta, norm_weight), ...)`` in one launch,
    without changing ``h``: ``h_out`` (when given) receives ``h + delta``.
    ``h``/``delta`` ``[T, n_tok, hidden]`` bf16.  Identical values to the two
    launches; None when the shape is outside the kernel's range."""
    dev = _lib.require_gpu(h, delta, norm_weight, w_packed, beta, threshold, out, h_out)
    _norm_inputs(h, delta, norm_weight, h_out, "norm_mlp_gate_lif")
    if h.ndim != 3:
        raise ValueError("norm_mlp_gate_lif: h must be [T, n_tok, hidden]")
    T, n, hidden = h.shape
    I = beta.numel()
    if threshold.numel() != I or w_packed.numel() * w_packed.element_size() != 4 * I * hidden:
        raise ValueError(f"packed weight / beta / threshold do not match hidden={hidden}, I={I}")
    if out is None:
        out = torch.empty((T, n, I), dtype=h.dtype, device=dev)
    elif tuple(out.shape) != (T, n, I) or not out.is_contiguous() or out.dtype != h.dtype:
        raise ValueError(f"out must be contiguous bf16 [{T}, {n}, {I}]")
    beta = beta.float().contiguous()
    threshold = threshold.float().contiguous()
    rc = _lib.load().spk_norm_mlp_gate_lif(
        h.data_ptr(), delta.data_ptr(), norm_weight.data_ptr(), _lib.ptr(h_out), float(eps),
        w_packed.data_ptr(), beta.data_ptr(), threshold.data_ptr(), _lib.dtype_code(beta.dtype),
        out.data_ptr(), T, n, hidden, I, _lib.dtype_code(h.dtype), _lib.stream_of(dev))
    if rc == _lib.SPK_EUNSUPPORTED:
        return None
    _lib.check(rc, "norm_mlp_gate_lif")
    return out


def decode_advance(next_tokens, input_ids, positions, seq_lens, slot_mapping, block_tables,
                   block_size: int, n_rows: int, live=None, history=None, step=None,
                   rng_seeds=None, uniforms=None) -> None:
    """Moves rows ``[0, n_live)`` of a decode batch to their next token on the
    device (no host sync); ``n_live = min(n_rows, live[0])`` when the int32
    device count ``live`` is given, else ``n_rows``.  With ``rng_seeds`` (int64
    ``[n_rows]``) and ``uniforms`` (fp32 ``[n_rows]``) it also writes each
    row's draw for the next step (a function of its seed and the step count)."""
    dev = _lib.require_gpu(next_tokens, input_ids, positions, seq_lens, slot_mapping, block_tables,
                           live, history, step, rng_seeds, uniforms)
    if live is not None and live.dtype != torch.int32:
        raise ValueError("live must be an int32 device count")
    for name, t, dt in (("next_tokens", next_tokens, torch.int64), ("input_ids", input_ids, torch.int64),
                        ("positions", positions, torch.int64), ("seq_lens", seq_lens, torch.int32),
                        ("slot_mapping", slot_mapping, torch.int64),
                        ("block_tables", block_tables, torch.int32)):
        if t.dtype != dt:
            raise ValueError(f"{name} must be {dt}")
        if t.ndim == 1 and not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if uniforms is not None:
        if (rng_seeds is None or step is None or rng_seeds.dtype != torch.int64
                or uniforms.dtype != torch.float32 or rng_seeds.numel() < n_rows
                or uniforms.numel() < n_rows or not rng_seeds.is_contiguous()
                or not uniforms.is_contiguous()):
            raise ValueError("uniforms need contiguous int64 rng_seeds and fp32 uniforms of n_rows "
                             "entries and a step counter")
    hist_cap = 0
    if history is not None:
        if step is None or history.dtype != torch.int64 or not history.is_contiguous():
            raise ValueError("history must be contiguous int64 [rows, cap] with an int32 step counter")
        hist_cap = history.shape[1]
    _lib.check(
        _lib.load().spk_decode_advance(
            next_tokens.data_ptr(), input_ids.data_ptr(), positions.data_ptr(), seq_lens.data_ptr(),
            slot_mapping.data_ptr(), block_tables.data_ptr(), block_tables.stride(0),
            block_tables.stride(1), block_tables.shape[1], block_size, n_rows,
            _lib.ptr(live), _lib.ptr(history), _lib.ptr(step), hist_cap, _lib.ptr(rng_seeds),
            _lib.ptr(uniforms), _lib.stream_of(dev),
        ),
        "decode_advance",
    )
