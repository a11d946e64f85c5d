"""Spiking Qwen2-architecture decoder on the HIP operators (whole-step decode).

Counterpart of spikeinfer/modeling_fast.py (FastSpikingQwenForCausalLM), with
the same flattened, paged forward: ``forward_paged(input_ids, positions,
kv_caches, meta)`` over ``[n_tok]`` tokens, decodes first, T residual streams
carried as one ``[T, n_tok, hidden]`` tensor so every GEMM has M = T * n_tok
(modeling_fast.py:265-319).

MI355X layout of a layer:
  * q/k/v projections are one GEMM on the concatenated weight ``[(Hq + 2 Hkv)
    D, hidden]``; at decode its output feeds the attention kernel itself
    (qkv_decode_attention: RoPE -> LIF -> pack of its heads, k/v written to
    their cache slots, then the decode attention), at prefill one kernel doing
    RoPE -> LIF -> pack and the cache write;
  * gate and up are one GEMM on ``[2 I, hidden]`` fused with the gate LIF and
    the product with up (mlp_gate_lif) at decode sizes;
  * each residual add is fused into the RMSNorm that follows it; the final
    norm is fused with the rate-coded mean over T.  (``fused_norm`` also moves
    the add + norm into the prologue of the GEMM that consumes it; it is off
    by default, being slower.)
At decode sizes the GEMMs are this package's kernels (linear_decode,
mlp_gate_lif), except the down projection above ``small_down_max_rows``
rows; larger batches (prefill) use torch's library GEMMs.
Weights load from the reference's parameter names
(:meth:`SpikingDecoder.load_reference_state_dict`).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .attention import AttentionMetadata
from .kernels.decoder_ops import (add_rmsnorm, embed_rmsnorm, lif_gate_mul, linear_decode,
                                  mlp_gate_lif, norm_linear_decode, norm_mlp_gate_lif, pack_gate_up,
                                  pack_linear, qkv_decode_attention, qkv_rope_lif_pack, rmsnorm_mean_t)
from .kernels.packing import packed_width
from .kernels.spike_attention import gather_kv_unpacked_pair, paged_spike_attn_decode


@dataclass
class SpikingQwenConfig:
    """The fields of SpikingQwenConfig (reference/modeling_spiking_qwen.py:28-35,
    a Qwen2Config) that the forward reads; defaults are Qwen2.5-0.5B's."""

    vocab_size: int = 151936
    hidden_size: int = 896
    intermediate_size: int = 4864
    num_hidden_layers: int = 24
    num_attention_heads: int = 14
    num_key_value_heads: int = 2
    head_dim: int = 64
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    tie_word_embeddings: bool = True
    max_position_embeddings: int = 32768
    T: int = 4
    beta_init: float = 0.9
    threshold_init: float = 1.0


class _Layer:
    __slots__ = ("input_norm", "post_norm", "w_qkv", "b_qkv", "lif_qkv_beta", "lif_qkv_th",
                 "w_o", "w_gu", "lif_gate_beta", "lif_gate_th", "w_down", "w_gu_packed",
                 "w_qkv_packed", "w_o_packed", "w_down_packed")


class SpikingDecoder:
    """Random-init (or reference-loaded) weights plus the paged forward."""

    def __init__(self, config: SpikingQwenConfig, device="cuda", dtype=torch.bfloat16,
                 seed: int = 0, init_std: float = 0.02) -> None:
        c = self.config = config
        self.device = torch.device(device)
        self.dtype = dtype
        self.T = c.T
        self.Hq, self.Hkv, self.D = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        self.W = packed_width(self.D)
        g = torch.Generator(device=self.device).manual_seed(seed)

        def normal(*shape):
            return torch.empty(shape, device=self.device, dtype=dtype).normal_(0.0, init_std, generator=g)

        def const(v, *shape):
            return torch.full(shape, v, device=self.device, dtype=dtype)

        H, I = c.hidden_size, c.intermediate_size
        C = (self.Hq + 2 * self.Hkv) * self.D
        self.embed = normal(c.vocab_size, H)
        self.lm_head = self.embed if c.tie_word_embeddings else normal(c.vocab_size, H)
        self.final_norm = const(1.0, H)
        self.layers: list[_Layer] = []
        for _ in range(c.num_hidden_layers):
            L = _Layer()
            L.input_norm = const(1.0, H)
            L.post_norm = const(1.0, H)
            L.w_qkv = normal(C, H)
            L.b_qkv = normal(C)
            # q/k/v LIF parameters: the model-dtype values, kept in fp32 (exact) because
            # the fused decode kernel reads fp32
            L.lif_qkv_beta = const(c.beta_init, 3, self.D).float()
            L.lif_qkv_th = const(c.threshold_init, 3, self.D).float()
            L.w_o = normal(H, self.Hq * self.D)
            L.w_gu = normal(2 * I, H)
            L.lif_gate_beta = const(c.beta_init, I).float()  # model-dtype values in fp32
            L.lif_gate_th = const(c.threshold_init, I).float()
            L.w_down = normal(H, I)
            self.layers.append(L)
        # Decode-only batches run q/k/v spikes and attention as one launch
        # (qkv_decode_attention); False keeps the two launches (same results).
        self.fused_attention = True
        # Batches of at most fused_mlp_max_tokens tokens run the gate|up GEMM,
        # the gate LIF and the product as one launch (mlp_gate_lif, from a
        # repacked copy of w_gu); False keeps the GEMM + lif_gate_mul.
        self.fused_mlp = True
        self.fused_mlp_max_tokens = 64
        # The same batches run the q/k/v and o projections through
        # linear_decode (repacked copies of w_qkv, w_o); False keeps F.linear.
        # The down projection (long K) goes there only up to small_down_max_rows
        # rows (T * tokens): beyond, the library GEMM is faster.
        self.small_linear = True
        self.small_down_max_rows = 128
        # True folds each residual add + RMSNorm into the GEMM that consumes
        # its output (norm_linear_decode for q/k/v, norm_mlp_gate_lif for the
        # MLP): two launches fewer a layer, identical values, the residual
        # stream alternating between two buffers.  Off: every workgroup of a
        # row group recomputes its rows' norm (64 column ranges share a row
        # group), which costs more than the launches it saves (config 5: 2.28
        # against 1.63 ms a step).
        self.fused_norm = False
        self._pack_mlp()
        # Rotary inverse frequencies as Qwen2RotaryEmbedding builds them (fp32, host).
        exps = torch.arange(0, self.D, 2, dtype=torch.int64).float() / self.D
        self.inv_freq = (1.0 / (c.rope_theta ** exps)).to(self.device)
        # cos/sin of every position, computed once by the same ops as
        # rope_tables (so a table row equals the per-step value bit for bit);
        # the q/k/v kernel reads row positions[i] for token i.
        with torch.no_grad():
            self.rope_cos, self.rope_sin = self.rope_tables(
                torch.arange(c.max_position_embeddings, device=self.device))

    # -- weights -----------------------------------------------------------
    def load_reference_state_dict(self, sd: dict[str, torch.Tensor]) -> None:
        """Loads FastSpikingQwenForCausalLM parameter names
        (modeling_fast.py:102-117, :180-200, :219-225, :322-329)."""
        cast = lambda t: t.to(self.device, self.dtype)
        self.embed = cast(sd["model.embed_tokens.weight"])
        self.lm_head = self.embed if self.config.tie_word_embeddings else cast(sd["lm_head.weight"])
        self.final_norm = cast(sd["model.norm.weight"])
        for i, L in enumerate(self.layers):
            p = f"model.layers.{i}."
            a, m = p + "self_attn.", p + "mlp."
            L.input_norm = cast(sd[p + "input_layernorm.weight"])
            L.post_norm = cast(sd[p + "post_attention_layernorm.weight"])
            L.w_qkv = cast(torch.cat([sd[a + f"{s}_proj.weight"] for s in "qkv"]))
            L.b_qkv = cast(torch.cat([sd[a + f"{s}_proj.bias"] for s in "qkv"]))
            L.lif_qkv_beta = cast(torch.stack([sd[a + f"lif_{s}.lif.beta"] for s in "qkv"])).float()
            L.lif_qkv_th = cast(torch.stack([sd[a + f"lif_{s}.lif.threshold"] for s in "qkv"])).float()
            L.w_o = cast(sd[a + "o_proj.weight"])
            L.w_gu = cast(torch.cat([sd[m + "gate_proj.weight"], sd[m + "up_proj.weight"]]))
            L.lif_gate_beta = cast(sd[m + "lif_gate.lif.beta"]).float()
            L.lif_gate_th = cast(sd[m + "lif_gate.lif.threshold"]).float()
            L.w_down = cast(sd[m + "down_proj.weight"])
        self._pack_mlp()

    def _pack_mlp(self) -> None:
        """Operand-order copies of w_gu (fused MLP gate) and of w_qkv, w_o and
        the lm_head (linear_decode); bf16 only."""
        self.lm_head_packed = None
        if self.dtype == torch.bfloat16:
            try:
                self.lm_head_packed = pack_linear(self.lm_head)
            except ValueError:
                pass
        for L in self.layers:
            L.w_gu_packed = L.w_qkv_packed = L.w_o_packed = L.w_down_packed = None
            if self.dtype != torch.bfloat16:
                continue
            for name, fn in (("w_gu", pack_gate_up), ("w_qkv", pack_linear), ("w_o", pack_linear),
                             ("w_down", pack_linear)):
                try:
                    setattr(L, name + "_packed", fn(getattr(L, name)))
                except ValueError:
                    pass

    def _linear(self, x: torch.Tensor, w: torch.Tensor, b, wp, n: int) -> torch.Tensor:
        """F.linear, or linear_decode for batches of at most fused_mlp_max_tokens."""
        if self.small_linear and wp is not None and n <= self.fused_mlp_max_tokens:
            y = linear_decode(x, wp, b)
            if y is not None:
                return y
        return F.linear(x, w, b)

    @property
    def weight_bytes(self) -> int:
        """Bytes of weights one decode step reads (tied lm_head counted once
        as the head, the embedding gather aside)."""
        n = self.lm_head.numel() + self.final_norm.numel()
        for L in self.layers:
            for name in _Layer.__slots__:
                if not name.endswith("_packed"):  # a step reads these instead of the originals
                    n += getattr(L, name).numel()
        return n * self.lm_head.element_size()

    # -- forward -----------------------------------------------------------
    def rope_tables(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """cos/sin ``[n_tok, D]`` in the model dtype, computed as
        Qwen2RotaryEmbedding does (fp32 outer product, cat, cos/sin, cast)."""
        freqs = positions.float()[:, None] * self.inv_freq[None, :]
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(self.dtype), emb.sin().to(self.dtype)

    def forward_paged(self, input_ids: torch.Tensor, positions: torch.Tensor,
                      kv_caches, meta: AttentionMetadata, bufs: dict | None = None) -> torch.Tensor:
        """``[n_tok]`` tokens (decodes first) -> ``[n_tok, hidden]`` rate-coded
        hidden states, writing every token's K/V into ``kv_caches[i] = (k, v)``.

        ``bufs`` optionally supplies preallocated ``q_packed`` ``[T, n_dec, Hq,
        W]`` and ``attn`` ``[T, n_tok, Hq, D]`` (stable addresses under graph
        capture).
        """
        c = self.config
        T, n = self.T, input_ids.shape[0]
        H, D, Hq, Hkv = c.hidden_size, self.D, self.Hq, self.Hkv
        n_dec = meta.num_decode_tokens
        bufs = bufs or {}
        positions = positions.to(torch.int64).contiguous()
        h, x = embed_rmsnorm(input_ids, self.embed, self.layers[0].input_norm, c.rms_norm_eps, T)
        q_packed = bufs.get("q_packed")
        if n_dec and q_packed is None:
            q_packed = torch.empty((T, n_dec, Hq, self.W), dtype=torch.int32, device=h.device)
        attn = bufs.get("attn")
        if attn is None:
            attn = torch.empty((T, n, Hq, D), dtype=self.dtype, device=h.device)
        dense = None
        if meta.num_prefills:
            dense = (torch.empty((T, Hq, n, D), dtype=self.dtype, device=h.device),
                     torch.empty((T, Hkv, n, D), dtype=self.dtype, device=h.device),
                     torch.empty((T, Hkv, n, D), dtype=self.dtype, device=h.device))
        delta = None
        fold = (self.fused_norm and self.small_linear and n <= self.fused_mlp_max_tokens
                and self.dtype == torch.bfloat16)
        h_alt = torch.empty_like(h) if fold else None  # the other residual buffer
        for i, L in enumerate(self.layers):
            k_cache, v_cache = kv_caches[i]
            qkv = None
            if i and fold and L.w_qkv_packed is not None:
                qkv = norm_linear_decode(h, delta, L.input_norm, c.rms_norm_eps, L.w_qkv_packed, L.b_qkv,
                                         h_out=h_alt)
                if qkv is not None:
                    h, h_alt = h_alt, h
            if qkv is None:
                if i:
                    x = add_rmsnorm(h, delta, L.input_norm, c.rms_norm_eps, out=x)
                qkv = self._linear(x, L.w_qkv, L.b_qkv, L.w_qkv_packed, n)
            fused = (self.fused_attention and not meta.num_prefills and n_dec == n and
                     qkv_decode_attention(qkv, self.rope_cos, self.rope_sin, positions, L.lif_qkv_beta,
                                          L.lif_qkv_th, k_cache, v_cache, meta.slot_mapping,
                                          meta.block_tables, meta.seq_lens, Hq, Hkv, meta.block_size,
                                          attn))
            if not fused:
                qkv_rope_lif_pack(qkv, self.rope_cos, self.rope_sin, L.lif_qkv_beta, L.lif_qkv_th,
                                  k_cache, v_cache, meta.slot_mapping, Hq, Hkv, D, q_packed=q_packed,
                                  n_q=n_dec, dense=dense, positions=positions)
            if n_dec and not fused:
                paged_spike_attn_decode(q_packed, k_cache, v_cache, meta.block_tables, meta.seq_lens,
                                        head_dim=D, block_size=meta.block_size, num_q_heads=Hq,
                                        num_kv_heads=Hkv, out=attn[:, :n_dec])
            if meta.num_prefills:
                self._prefill_attention(dense, k_cache, v_cache, meta, attn)
            o = self._linear(attn.view(T, n, Hq * D), L.w_o, None, L.w_o_packed, n)
            y = None
            if fold and self.fused_mlp and L.w_gu_packed is not None:
                y = norm_mlp_gate_lif(h, o, L.post_norm, c.rms_norm_eps, L.w_gu_packed, L.lif_gate_beta,
                                      L.lif_gate_th, h_out=h_alt)
                if y is not None:
                    h, h_alt = h_alt, h
            if y is None:
                x = add_rmsnorm(h, o, L.post_norm, c.rms_norm_eps, out=x)
            if y is None and self.fused_mlp and L.w_gu_packed is not None and n <= self.fused_mlp_max_tokens:
                y = mlp_gate_lif(x, L.w_gu_packed, L.lif_gate_beta, L.lif_gate_th)
            if y is None:
                y = lif_gate_mul(F.linear(x, L.w_gu), L.lif_gate_beta, L.lif_gate_th)
            delta = None
            if T * n <= self.small_down_max_rows:
                delta = self._linear(y, L.w_down, None, L.w_down_packed, n)
            if delta is None:
                delta = F.linear(y, L.w_down)
        return rmsnorm_mean_t(h, self.final_norm, c.rms_norm_eps, delta=delta)

    def _prefill_attention(self, dense, k_cache, v_cache, meta: AttentionMetadata, attn) -> None:
        """Prefill chunks (attention.py:161-178): SDPA on the chunk's dense
        query spikes against its whole cached prefix.  A chunk with no cached
        prefix attends to its own dense k/v spikes (identical to what was just
        written to the cache); equal-length fresh chunks go in one batched call."""
        dq, dk, dv = dense
        T, D, Hq = self.T, self.D, self.Hq
        chunks = list(zip(meta.prefill_query_starts, meta.prefill_query_lens,
                          meta.prefill_context_lens, meta.prefill_block_tables))
        fresh = [ch for ch in chunks if ch[2] == 0]
        if fresh and len({ch[1] for ch in fresh}) == 1 and \
                all(fresh[j + 1][0] == fresh[j][0] + fresh[j][1] for j in range(len(fresh) - 1)):
            s0, L, B = fresh[0][0], fresh[0][1], len(fresh)

            def batch(t, heads):
                return t[:, :, s0:s0 + B * L].reshape(T, heads, B, L, D).transpose(1, 2).reshape(T * B, heads, L, D)

            o = F.scaled_dot_product_attention(batch(dq, Hq), batch(dk, self.Hkv), batch(dv, self.Hkv),
                                               is_causal=True, enable_gqa=Hq != self.Hkv)
            attn[:, s0:s0 + B * L] = o.view(T, B, Hq, L, D).permute(0, 1, 3, 2, 4).reshape(T, B * L, Hq, D)
            chunks = [ch for ch in chunks if ch not in fresh]
        for start, q_len, ctx, table in chunks:
            total = ctx + q_len
            if ctx == 0:
                k_all, v_all = dk[:, :, start:start + q_len], dv[:, :, start:start + q_len]
            else:
                k_all, v_all = gather_kv_unpacked_pair(k_cache, v_cache, table, total, D,
                                                       meta.block_size, self.dtype)
            mask = torch.full((q_len, total), float("-inf"), device=attn.device, dtype=self.dtype)
            mask = torch.triu(mask, diagonal=ctx + 1)
            o = F.scaled_dot_product_attention(dq[:, :, start:start + q_len], k_all, v_all,
                                               attn_mask=mask, enable_gqa=Hq != self.Hkv)
            attn[:, start:start + q_len] = o.permute(0, 2, 1, 3)

    def compute_logits(self, hidden: torch.Tensor, indices: torch.Tensor | None = None,
                       out: torch.Tensor | None = None) -> torch.Tensor:
        """lm_head on the rows that sample (modeling_fast.py:335-355)."""
        if indices is not None:
            hidden = hidden.index_select(0, indices)
        if self.small_linear and self.lm_head_packed is not None and hidden.shape[0] <= 64:
            y = linear_decode(hidden, self.lm_head_packed, None, out)
            if y is not None:
                return y
        if out is None:
            return F.linear(hidden, self.lm_head)
        return torch.matmul(hidden, self.lm_head.t(), out=out)
