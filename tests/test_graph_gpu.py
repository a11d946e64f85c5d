"""hipGraph capture of the fused LIF-pack-write and the decode attention.

The captured graph is replayed several times with eager work and
synchronisations in between; every replay must equal the eager result
(capture safety: no host sync, no allocation outside torch's graph pool).
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_capture_lif_pack_write_and_decode(gpu):
    from spikeinfer_amd.kernels import lif_pack_write, paged_spike_attn_decode

    torch.manual_seed(0)
    T, N, Hq, Hkv, D, bs, max_blocks = 4, 8, 14, 2, 64, 16, 400
    num_blocks = N * max_blocks + 1
    k_cache = torch.zeros((T, Hkv, num_blocks * bs, 2), dtype=torch.int32, device=gpu)
    v_cache = torch.zeros_like(k_cache)
    # fill caches with random packed spikes
    k_cache.copy_(torch.randint(-2**31, 2**31 - 1, k_cache.shape, dtype=torch.int32, device=gpu))
    v_cache.copy_(torch.randint(-2**31, 2**31 - 1, v_cache.shape, dtype=torch.int32, device=gpu))
    tables = torch.randperm(num_blocks - 1, device=gpu)[: N * max_blocks].view(N, max_blocks).int()
    lens = torch.randint(1, max_blocks * bs, (N,), device=gpu, dtype=torch.int32)
    beta = torch.rand(D, device=gpu)
    th = torch.rand(D, device=gpu) * 0.5 + 0.1
    x_q = torch.randn(T, N, Hq, D, device=gpu, dtype=torch.bfloat16)
    x_k = torch.randn(T, N, Hkv, D, device=gpu, dtype=torch.bfloat16)
    slots = (tables[:, 0].long() * bs)
    q_buf = torch.zeros((T, N, Hq, 2), dtype=torch.int32, device=gpu)
    out = torch.empty((T, N, Hq, D), device=gpu, dtype=torch.float32)

    def body():
        lif_pack_write(x_q, beta, th, q_buf)
        lif_pack_write(x_k, beta, th, k_cache, slot_mapping=slots)
        paged_spike_attn_decode(q_buf, k_cache, v_cache, tables, lens, D, bs, Hq, Hkv, out=out)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            body()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        body()

    for it in range(4):
        x_q.copy_(torch.randn_like(x_q))
        x_k.copy_(torch.randn_like(x_k))
        lens.copy_(torch.randint(1, max_blocks * bs, (N,), device=gpu, dtype=torch.int32))
        torch.cuda.synchronize()
        k_before = k_cache.clone()
        g.replay()
        torch.cuda.synchronize()
        got, got_q, got_k = out.clone(), q_buf.clone(), k_cache.clone()
        k_cache.copy_(k_before)
        body()  # eager
        torch.cuda.synchronize()
        assert torch.equal(got_q, q_buf), f"replay {it}: q buffer differs"
        assert torch.equal(got_k, k_cache), f"replay {it}: cache differs"
        assert torch.equal(got, out), f"replay {it}: attention differs"


def test_capture_dense_lif_multistep_as_the_graphed_decoder_uses_it(gpu):
    """The dense LIF sites of one decode step as GraphedDecoder captures them
    (spikeinfer/graph_runner.py:110-129 -> modeling_fast.py:121-135, :186-190):
    q/k/v on the permuted [T, B, H, S, D] projection views (the wrapper's
    reshape copies them), the MLP gate on [T, B, S, I]; four replays with new
    currents, each equal to an eager run."""
    from spikeinfer_amd.kernels import lif_multistep

    torch.manual_seed(1)
    T, B, S, Hq, Hkv, D, I = 4, 8, 1, 14, 2, 64, 4864
    q_lin = torch.randn(T, B, S, Hq * D, device=gpu, dtype=torch.bfloat16)
    k_lin = torch.randn(T, B, S, Hkv * D, device=gpu, dtype=torch.bfloat16)
    g_lin = torch.randn(T, B, S, I, device=gpu, dtype=torch.bfloat16)
    bq, tq = torch.rand(D, device=gpu), torch.rand(D, device=gpu) + 0.2
    bg, tg = torch.rand(I, device=gpu), torch.rand(I, device=gpu) + 0.2
    outs = {}

    def body():
        q = q_lin.view(T, B, S, Hq, D).permute(0, 1, 3, 2, 4)
        k = k_lin.view(T, B, S, Hkv, D).permute(0, 1, 3, 2, 4)
        outs["q"] = lif_multistep(q, bq, tq)
        outs["k"] = lif_multistep(k, bq, tq)
        outs["g"] = lif_multistep(g_lin, bg, tg)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            body()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        body()
    graph_outs = dict(outs)
    for it in range(4):
        for t in (q_lin, k_lin, g_lin):
            t.copy_(torch.randn_like(t))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = {k: v.clone() for k, v in graph_outs.items()}
        body()
        torch.cuda.synchronize()
        for name in got:
            assert got[name].shape == outs[name].shape
            assert torch.equal(got[name], outs[name]), f"replay {it}: {name} differs"
