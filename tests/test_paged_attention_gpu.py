"""The attention step over the paged spike cache (spikeinfer/attention.py:111-180).

Restates the reference's conventions on a mixed batch: decodes first, then
prefill chunks; the step's K/V are written before anyone attends; ``seq_lens``
include the token being decoded; graph pad rows point at the pad block with
``seq_len = 1`` (engine/model_runner.py:234-240).  Expected values come from the
CPU oracle: packed cache bytes bit-exact; decode rows from the C decode oracle,
prefill rows from the float64 prefill oracle.

Tolerances (max abs on outputs in [0, 1]): fp32 1e-3 (decode kernel; SDPA on
exact 0/1 operands is far tighter); bf16 outputs 2**-7 + 1e-3, since SDPA rounds
its probabilities and output to bf16 for prefill rows.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from spikeinfer_amd.attention import AttentionMetadata, paged_attention, paged_attention_fused
from spikeinfer_amd.kernels import lif_multistep
from spikeinfer_amd.spike_cache import PagedSpikeCache, slot_mapping

pytestmark = pytest.mark.gpu

T, HQ, HKV, D, BS = 4, 14, 2, 64, 16
TOL = {torch.float32: 1e-3, torch.bfloat16: 2.0**-7 + 1e-3, torch.float16: 2.0**-10 + 1e-3}


def _build_step(seed, dec_lens, prefills, num_blocks=64, pad_rows=0, device="cuda"):
    """A cache pre-filled with random history and a mixed batch.

    dec_lens: seq_len of each decode row (its new token sits at seq_len - 1).
    prefills: (context_len, q_len) of each prefill chunk.
    Returns (cache, meta, host-side description).
    """
    rng = np.random.default_rng(seed)
    cache = PagedSpikeCache(1, T, HKV, D, num_blocks, BS, device=device)
    k0 = orc.pack((rng.random(tuple(cache.k[0].shape[:3]) + (D,)) < 0.3).astype(np.uint8))
    v0 = orc.pack((rng.random(tuple(cache.v[0].shape[:3]) + (D,)) < 0.3).astype(np.uint8))
    cache.k[0].copy_(torch.from_numpy(k0))
    cache.v[0].copy_(torch.from_numpy(v0))

    free = list(rng.permutation(cache.num_allocatable_blocks))
    def alloc(n_tok):
        need = (n_tok + BS - 1) // BS
        out = [int(free.pop()) for _ in range(need)]
        return out

    max_blocks = max([(L + BS - 1) // BS for L in dec_lens] + [1])
    tables, slots, lens = [], [], []
    for L in dec_lens:
        tab = alloc(L)
        tables.append(tab + [cache.pad_block] * (max_blocks - len(tab)))
        slots += slot_mapping(tab, L - 1, 1, BS)
        lens.append(L)
    for _ in range(pad_rows):
        tables.append([cache.pad_block] * max_blocks)
        slots.append(cache.pad_slot)
        lens.append(1)
    n_dec = len(dec_lens) + pad_rows
    starts, qlens, ctxs, ptabs = [], [], [], []
    cur = n_dec
    for ctx, q_len in prefills:
        tab = alloc(ctx + q_len)
        starts.append(cur)
        qlens.append(q_len)
        ctxs.append(ctx)
        ptabs.append(tab)
        slots += slot_mapping(tab, ctx, q_len, BS)
        cur += q_len
    meta = AttentionMetadata(
        slot_mapping=torch.tensor(slots, dtype=torch.int64, device=device),
        block_size=BS,
        num_decode_tokens=n_dec,
        block_tables=torch.tensor(tables, dtype=torch.int32, device=device) if n_dec else None,
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=device) if n_dec else None,
        prefill_query_starts=starts,
        prefill_query_lens=qlens,
        prefill_context_lens=ctxs,
        prefill_block_tables=[torch.tensor(t, dtype=torch.int32, device=device) for t in ptabs],
    )
    host = dict(k0=k0, v0=v0, slots=np.array(slots, np.int64), tables=np.array(tables, np.int32)
                if n_dec else None, lens=np.array(lens, np.int32), n_tok=cur, n_dec=n_dec,
                prefills=list(zip(starts, qlens, ctxs, ptabs)))
    return cache, meta, host


def _scatter(cache0, slots, words, got):
    """cache0 with ``words[:, :, i]`` written at ``slots[i]``.  Where several
    tokens share a slot (graph pad rows all write the pad slot) index_copy_
    keeps one of them, unspecified which: check that the GPU kept one of the
    candidates and take that one."""
    want = cache0.copy()
    want[:, :, slots] = words
    uniq, counts = np.unique(slots, return_counts=True)
    for s in uniq[counts > 1]:
        cand = words[:, :, slots == s]  # [T, H, n_dup, W]
        kept = got[:, :, s]
        match = (cand == kept[:, :, None]).all(axis=-1).any(axis=-1)
        assert match.all(), f"slot {s} holds none of the values written to it"
        want[:, :, s] = kept
    return want


def _expected(host, q_bits, k_bits, v_bits, k_got, v_got):
    """Oracle for one step. *_bits: uint8 [T, H, n_tok, D]; *_got: the GPU caches."""
    k = _scatter(host["k0"], host["slots"], orc.pack(k_bits), k_got)
    v = _scatter(host["v0"], host["slots"], orc.pack(v_bits), v_got)
    out = np.zeros((T, host["n_tok"], HQ, D))
    n_dec = host["n_dec"]
    if n_dec:
        q = orc.pack(np.ascontiguousarray(q_bits[:, :, :n_dec].transpose(0, 2, 1, 3)))
        out[:, :n_dec] = orc.decode_attn(q, k, v, host["tables"], host["lens"], D, BS, HQ, HKV)
    for start, q_len, ctx, tab in host["prefills"]:
        o = orc.prefill_attn(q_bits[:, :, start:start + q_len], k, v, tab, ctx, D, BS, HQ, HKV)
        out[:, start:start + q_len] = o.transpose(0, 2, 1, 3)
    return k, v, out


def _bits(rng, H, n_tok, p=0.35):
    return (rng.random((T, H, n_tok, D)) < p).astype(np.uint8)


def _to_spikes(bits, dtype):
    return torch.from_numpy(bits).to("cuda", dtype).unsqueeze(1)  # [T, 1, H, n_tok, D]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize(
    "dec_lens,prefills,pad_rows",
    [
        ([37, 1, 300], [(0, 20), (33, 5)], 0),  # decodes, a fresh prompt, a later chunk
        ([17, 64, 65], [], 2),  # decode-only with graph pad rows
        ([], [(0, 48)], 0),  # prefill-only
        ([], [(16, 1), (100, 31)], 0),  # chunked prefill continuing a cached prefix
    ],
)
def test_paged_attention_matches_oracle(gpu, dtype, dec_lens, prefills, pad_rows):
    cache, meta, host = _build_step(7, dec_lens, prefills, pad_rows=pad_rows)
    rng = np.random.default_rng(11)
    n_tok = host["n_tok"]
    qb, kb, vb = _bits(rng, HQ, n_tok), _bits(rng, HKV, n_tok), _bits(rng, HKV, n_tok)
    out = paged_attention(_to_spikes(qb, dtype), _to_spikes(kb, dtype), _to_spikes(vb, dtype),
                          cache.k[0], cache.v[0], meta, HQ, HKV, D)
    torch.cuda.synchronize()
    k_got, v_got = cache.k[0].cpu().numpy(), cache.v[0].cpu().numpy()
    k_want, v_want, o_want = _expected(host, qb, kb, vb, k_got, v_got)
    assert np.array_equal(k_got, k_want)
    assert np.array_equal(v_got, v_want)
    assert out.shape == (T, 1, n_tok, HQ * D) and out.dtype == dtype
    got = out.float().view(T, n_tok, HQ, D).cpu().numpy()
    err = np.abs(got - o_want).max()
    assert err <= TOL[dtype], f"max abs err {err}"


def test_pad_rows_see_only_their_own_token(gpu):
    """A pad row (pad slot, pad-block table, seq_len 1) attends to exactly the
    value it wrote: its output is its own V bits, whatever else is cached."""
    cache, meta, host = _build_step(5, [40], [], pad_rows=3)
    rng = np.random.default_rng(2)
    qb, kb, vb = _bits(rng, HQ, 4), _bits(rng, HKV, 4), _bits(rng, HKV, 4)
    out = paged_attention(_to_spikes(qb, torch.float32), _to_spikes(kb, torch.float32),
                          _to_spikes(vb, torch.float32), cache.k[0], cache.v[0], meta, HQ, HKV, D)
    got = out.view(T, 4, HQ, D).cpu().numpy()
    # The three pad rows share the pad slot and index_copy_ keeps one of their
    # writes, unspecified which, so compare against what the cache holds.
    pad_v = orc.unpack(cache.v[0][:, :, cache.pad_slot].cpu().numpy(), D)  # [T, HKV, D]
    for row in (1, 2, 3):
        np.testing.assert_array_equal(got[:, row], np.repeat(pad_v, HQ // HKV, axis=1))


def _lif_params(seed):
    g = torch.Generator().manual_seed(seed)
    beta = (0.5 + 0.5 * torch.rand(D, generator=g)).cuda()
    thr = (0.5 + torch.rand(D, generator=g)).cuda()
    return beta, thr


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_step_matches_oracle_and_unfused(gpu, dtype):
    """paged_attention_fused from the currents == LIF (oracle) -> the oracle step,
    and == lif_multistep + paged_attention on the GPU (caches and output
    bit-identical: same spikes, same packed bytes, same kernels)."""
    dec_lens, prefills = [50, 3, 129, 16], [(0, 9), (20, 4)]
    cache_a, meta, host = _build_step(9, dec_lens, prefills)
    cache_b, _, _ = _build_step(9, dec_lens, prefills)
    n_tok = host["n_tok"]
    g = torch.Generator().manual_seed(4)
    cur = {h: (torch.randn((T, n_tok, n, D), generator=g) * 1.2 + 0.4).to(dtype).cuda()
           for h, n in (("q", HQ), ("k", HKV), ("v", HKV))}
    params = {h: _lif_params(i) for i, h in enumerate("qkv")}

    out_f = paged_attention_fused(cur["q"], cur["k"], cur["v"], params["q"], params["k"],
                                  params["v"], cache_a.k[0], cache_a.v[0], meta, HQ, HKV, D)
    spk = {h: lif_multistep(cur[h], *params[h]).permute(0, 2, 1, 3).unsqueeze(1) for h in "qkv"}
    out_u = paged_attention(spk["q"], spk["k"], spk["v"], cache_b.k[0], cache_b.v[0], meta,
                            HQ, HKV, D)
    torch.cuda.synchronize()
    assert torch.equal(cache_a.k[0], cache_b.k[0]) and torch.equal(cache_a.v[0], cache_b.v[0])
    assert torch.equal(out_f, out_u)

    bits = {}
    for h in "qkv":
        x = cur[h].float().cpu().numpy()
        b, th = (p.float().cpu().numpy() for p in params[h])
        s, _ = orc.lif(x, b, th)
        bits[h] = np.ascontiguousarray((s != 0).astype(np.uint8).transpose(0, 2, 1, 3))
    k_got, v_got = cache_a.k[0].cpu().numpy(), cache_a.v[0].cpu().numpy()
    k_want, v_want, o_want = _expected(host, bits["q"], bits["k"], bits["v"], k_got, v_got)
    assert np.array_equal(k_got, k_want)
    assert np.array_equal(v_got, v_want)
    got = out_f.float().view(T, n_tok, HQ, D).cpu().numpy()
    assert np.abs(got - o_want).max() <= TOL[dtype]


def test_fused_decode_step_replays_in_graph(gpu):
    """The decode-only fused step captured once and replayed on fresh currents
    and a grown context matches eager every time (static out / q_packed)."""
    dec_lens = [33, 200, 1, 90]
    cache_g, meta, host = _build_step(13, dec_lens, [], pad_rows=1)
    cache_e, _, _ = _build_step(13, dec_lens, [], pad_rows=1)
    n = host["n_tok"]
    params = {h: _lif_params(10 + i) for i, h in enumerate("qkv")}
    static = {h: torch.zeros((T, n, hh, D), dtype=torch.bfloat16, device="cuda")
              for h, hh in (("q", HQ), ("k", HKV), ("v", HKV))}
    out = torch.empty((T, n, HQ, D), dtype=torch.bfloat16, device="cuda")
    q_packed = torch.empty((T, n, HQ, 2), dtype=torch.int32, device="cuda")

    def step(c, cache, o=None, qp=None):
        return paged_attention_fused(c["q"], c["k"], c["v"], params["q"], params["k"],
                                     params["v"], cache.k[0], cache.v[0], meta, HQ, HKV, D,
                                     out=o, q_packed=qp)

    step(static, cache_g, out, q_packed)  # warm-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(static, cache_g, out, q_packed)
    g = torch.Generator().manual_seed(21)
    for rep in range(4):
        fresh = {h: torch.randn(static[h].shape, generator=g).to(torch.bfloat16).cuda()
                 for h in static}
        # Advance the real rows by one token: new slot, longer seq_len.
        if rep:
            meta.seq_lens[:len(dec_lens)] += 1
            lens = meta.seq_lens[:len(dec_lens)].cpu().tolist()
            tabs = meta.block_tables[:len(dec_lens)].cpu().tolist()
            new_slots = [tabs[i][(L - 1) // BS] * BS + (L - 1) % BS for i, L in enumerate(lens)]
            meta.slot_mapping[:len(dec_lens)] = torch.tensor(new_slots, device="cuda")
        for h in static:
            static[h].copy_(fresh[h])
        graph.replay()
        want = step(fresh, cache_e)
        torch.cuda.synchronize()
        assert torch.equal(out.view_as(want), want), f"replay {rep}"
        assert torch.equal(cache_g.k[0], cache_e.k[0]) and torch.equal(cache_g.v[0], cache_e.v[0])
