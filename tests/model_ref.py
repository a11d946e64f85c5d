"""Torch-only restatement of the reference's paged spiking forward, for tests.

Follows spikeinfer/modeling_fast.py:89-99 (RoPE by broadcast), :121-135
(spike_qkv), :186-190 (MLP), :206-211 (decoder layer), :265-319
(forward_paged); spikeinfer/attention.py:111-180 (paged_attention);
lif_triton.py:126-138 (lif_multistep_ref); packing.py:16-23 (bit layout);
spike_attention.py:224-282 (unpack-gather + SDPA decode oracle); transformers
Qwen2RMSNorm.  Separate q/k/v and gate/up projections, as the reference
model has them.  Uses no HIP kernel of this package, so it checks them.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def rms_norm(h, w, eps):
    x = h.to(torch.float32)
    var = x.pow(2).mean(-1, keepdim=True)
    x = x * torch.rsqrt(var + eps)
    return w * x.to(h.dtype)


def rotate_half(x):
    d = x.shape[-1] // 2
    return torch.cat((-x[..., d:], x[..., :d]), dim=-1)


def lif_ref(x, beta, threshold):
    b = beta.clamp(0, 1).to(torch.float32)
    th = threshold.to(torch.float32)
    u = torch.zeros(x.shape[1:], device=x.device, dtype=torch.float32)
    out = torch.empty_like(x)
    for t in range(x.shape[0]):
        r = (u - th > 0).to(torch.float32)
        u = b * u + x[t].to(torch.float32) - r * th
        out[t] = (u - th > 0).to(x.dtype)
    return out


def pack_ref(x):
    """[..., C] -> int32 [..., ceil(C/32)], bit i of word w = channel 32w + i."""
    C = x.shape[-1]
    W = (C + 31) // 32
    bits = (x != 0).to(torch.int64)
    if W * 32 != C:
        bits = F.pad(bits, (0, W * 32 - C))
    bits = bits.view(*x.shape[:-1], W, 32)
    words = (bits << torch.arange(32, device=x.device)).sum(-1)
    return ((words + 2**31) % 2**32 - 2**31).to(torch.int32)


def unpack_ref(words, C, dtype):
    bits = (words.to(torch.int64)[..., None] >> torch.arange(32, device=words.device)) & 1
    return bits.reshape(*words.shape[:-1], -1)[..., :C].to(dtype)


def gather_ref(cache, table, length, D, bs, dtype):
    pos = torch.arange(length, device=cache.device)
    slots = table.to(torch.int64)[pos // bs] * bs + pos % bs
    return unpack_ref(cache.index_select(2, slots), D, dtype)


def paged_attention_ref(q_spk, k_spk, v_spk, k_cache, v_cache, meta, Hq, Hkv, D):
    T, n = q_spk.shape[0], q_spk.shape[3]
    dtype = q_spk.dtype
    k_cache.index_copy_(2, meta.slot_mapping, pack_ref(k_spk.squeeze(1)))
    v_cache.index_copy_(2, meta.slot_mapping, pack_ref(v_spk.squeeze(1)))
    out = torch.empty((T, n, Hq, D), device=q_spk.device, dtype=dtype)
    rep = Hq // Hkv
    for i in range(meta.num_decode_tokens):
        L = int(meta.seq_lens[i])
        q = q_spk[:, 0, :, i].to(torch.float32)  # [T, Hq, D]
        k = gather_ref(k_cache, meta.block_tables[i], L, D, meta.block_size, torch.float32)
        v = gather_ref(v_cache, meta.block_tables[i], L, D, meta.block_size, torch.float32)
        k, v = k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1)
        o = F.scaled_dot_product_attention(q.unsqueeze(2), k, v)
        out[:, i] = o.squeeze(2).to(dtype)
    for start, q_len, ctx, table in zip(meta.prefill_query_starts, meta.prefill_query_lens,
                                        meta.prefill_context_lens, meta.prefill_block_tables):
        total = ctx + q_len
        k = gather_ref(k_cache, table, total, D, meta.block_size, dtype)
        v = gather_ref(v_cache, table, total, D, meta.block_size, dtype)
        q = q_spk[:, 0, :, start:start + q_len]
        mask = torch.triu(torch.full((q_len, total), float("-inf"), device=q.device, dtype=dtype),
                          diagonal=ctx + 1)
        o = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=Hq != Hkv)
        out[:, start:start + q_len] = o.permute(0, 2, 1, 3)
    return out.view(T, 1, n, Hq * D)


def forward_paged_ref(model, input_ids, positions, kv_caches, meta):
    """[n_tok] -> [n_tok, hidden], writing the caches, with the weights of a
    spikeinfer_amd.model.SpikingDecoder split back into the reference's
    separate projections."""
    c = model.config
    T, n, H = model.T, input_ids.shape[0], c.hidden_size
    Hq, Hkv, D, I = model.Hq, model.Hkv, model.D, c.intermediate_size
    cos, sin = model.rope_tables(positions)
    cos, sin = cos[None, None, None], sin[None, None, None]  # [1, 1, 1, n, D]
    h = F.embedding(input_ids, model.embed)[None].unsqueeze(0).expand(T, 1, n, H).contiguous()
    for i, L in enumerate(model.layers):
        x = rms_norm(h, L.input_norm, c.rms_norm_eps)
        w, b = L.w_qkv, L.b_qkv
        q = F.linear(x, w[:Hq * D], b[:Hq * D]).view(T, 1, n, Hq, D).permute(0, 1, 3, 2, 4)
        k = F.linear(x, w[Hq * D:(Hq + Hkv) * D], b[Hq * D:(Hq + Hkv) * D])
        v = F.linear(x, w[(Hq + Hkv) * D:], b[(Hq + Hkv) * D:])
        k = k.view(T, 1, n, Hkv, D).permute(0, 1, 3, 2, 4)
        v = v.view(T, 1, n, Hkv, D).permute(0, 1, 3, 2, 4)
        q, k = (q * cos) + (rotate_half(q) * sin), (k * cos) + (rotate_half(k) * sin)
        qs = lif_ref(q, L.lif_qkv_beta[0], L.lif_qkv_th[0])
        ks = lif_ref(k, L.lif_qkv_beta[1], L.lif_qkv_th[1])
        vs = lif_ref(v, L.lif_qkv_beta[2], L.lif_qkv_th[2])
        ctx = paged_attention_ref(qs, ks, vs, kv_caches[i][0], kv_caches[i][1], meta, Hq, Hkv, D)
        h = h + F.linear(ctx, L.w_o)
        x = rms_norm(h, L.post_norm, c.rms_norm_eps)
        gate = lif_ref(F.linear(x, L.w_gu[:I]), L.lif_gate_beta, L.lif_gate_th)
        h = h + F.linear(gate * F.linear(x, L.w_gu[I:]), L.w_down)
    return rms_norm(h, model.final_norm, c.rms_norm_eps).mean(dim=0).squeeze(0)
