"""HIP LIF / pack / fused LIF-pack-write vs the CPU oracle, bit-exact
(restates tests/test_lif_kernel.py and tests/test_packing.py of the reference).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _rand_beta(rng, n):
    return (rng.random(n) * 4.0 - 1.5).astype(np.float32)  # tests/test_lif_kernel.py:30-33


def _rand_th(rng, n):
    return (rng.random(n) * 0.95 + 0.05).astype(np.float32)


@pytest.mark.parametrize("M", [128, 1792])
@pytest.mark.parametrize("N", [64, 4864, 63])
@pytest.mark.parametrize("T", [1, 2, 4, 8])
def test_lif_multistep_bit_exact(T, N, M, gpu):
    """fp32 in/out: the 16-byte vector path for N % 4 == 0, scalar for N = 63."""
    from spikeinfer_amd.kernels import lif_multistep

    rng = np.random.default_rng(1000 * T + 10 * N + M)
    beta, th = _rand_beta(rng, N), _rand_th(rng, N)
    x = (rng.standard_normal((T, M, N)) * 2).astype(np.float32)
    print(f"lif T={T} N={N} M={M}", flush=True)
    s, u = lif_multistep(torch.from_numpy(x).to(gpu), torch.from_numpy(beta).to(gpu),
                         torch.from_numpy(th).to(gpu), return_membrane=True)
    ws, wu = orc.lif(x, beta, th)
    assert np.array_equal(s.cpu().numpy().astype(np.uint8), ws)
    assert np.array_equal(u.cpu().numpy().view(np.uint32), wu.view(np.uint32))


def test_lif_threshold_boundary_stress(gpu):
    from spikeinfer_amd.kernels import lif_multistep

    rng = np.random.default_rng(0)
    T, M, N = 8, 256, 64
    beta = np.full(N, 0.9, np.float32)
    th = np.full(N, 1.0, np.float32)
    x = (np.ones((T, M, N)) + rng.standard_normal((T, M, N)) * 1e-6).astype(np.float32)
    s, u = lif_multistep(torch.from_numpy(x).to(gpu), torch.from_numpy(beta).to(gpu),
                         torch.from_numpy(th).to(gpu), return_membrane=True)
    ws, wu = orc.lif(x, beta, th)
    assert np.array_equal(s.cpu().numpy().astype(np.uint8), ws), "FMA contraction regression?"
    assert np.array_equal(u.cpu().numpy(), wu)


@pytest.mark.parametrize("in_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("out_dtype", [None, torch.uint8, torch.float32, torch.bool])
def test_lif_dtypes_and_5d_noncontiguous(in_dtype, out_dtype, gpu):
    from spikeinfer_amd.kernels import lif_multistep

    rng = np.random.default_rng(42)
    T, B, S, H, D = 4, 2, 5, 3, 64
    beta, th = _rand_beta(rng, D), _rand_th(rng, D)
    base = torch.from_numpy(rng.standard_normal((T, B, S, H, D)).astype(np.float32)).to(gpu)
    x = base.to(in_dtype).permute(0, 1, 3, 2, 4)  # [T,B,H,S,D] view, as modeling_fast
    assert not x.is_contiguous()
    s = lif_multistep(x, torch.from_numpy(beta).to(gpu), torch.from_numpy(th).to(gpu),
                      out_dtype=out_dtype)
    assert s.dtype == (out_dtype or in_dtype) and s.shape == x.shape
    ws, _ = orc.lif(x.float().cpu().numpy(), beta, th)
    assert np.array_equal(s.to(torch.uint8).cpu().numpy(), ws)


def test_lif_mem0_and_bf16_params(gpu):
    from spikeinfer_amd.kernels import lif_multistep

    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 40, 96)).astype(np.float32)
    m0 = rng.standard_normal((40, 96)).astype(np.float32)
    beta = torch.from_numpy(_rand_beta(rng, 96)).to(gpu).bfloat16()
    th = torch.from_numpy(_rand_th(rng, 96)).to(gpu).bfloat16()
    s, u = lif_multistep(torch.from_numpy(x).to(gpu), beta, th, mem0=torch.from_numpy(m0).to(gpu),
                         return_membrane=True)
    ws, wu = orc.lif(x, beta.float().cpu().numpy(), th.float().cpu().numpy(), m0)
    assert np.array_equal(s.cpu().numpy().astype(np.uint8), ws)
    assert np.array_equal(u.cpu().numpy(), wu)


# ---- packing ---------------------------------------------------------------
@pytest.mark.parametrize("channels", [1, 31, 32, 33, 63, 64, 128, 256, 4864])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.uint8, torch.int32])
def test_pack_roundtrip_and_bytes(channels, dtype, gpu):
    from spikeinfer_amd.kernels import pack_spikes, unpack_spikes

    rng = np.random.default_rng(channels)
    bits = (rng.random((3, 5, channels)) > 0.5).astype(np.uint8)
    x = torch.from_numpy(bits).to(gpu).to(dtype)
    words = pack_spikes(x)
    assert words.dtype == torch.int32 and words.shape == (3, 5, (channels + 31) // 32)
    assert np.array_equal(words.cpu().numpy(), orc.np_pack(bits))
    assert torch.equal(unpack_spikes(words, channels, dtype), x)


def test_pack_known_answers(gpu):
    from spikeinfer_amd.kernels import pack_spikes, unpack_spikes

    assert pack_spikes(torch.ones(1, 32, device=gpu)).item() == -1
    assert int(pack_spikes(torch.ones(1, 33, device=gpu))[0, 1]) == 1
    g = pack_spikes(torch.tensor([[0.0, 0.5, 0.0, 2.0]], device=gpu))
    assert unpack_spikes(g, 4).tolist() == [[0.0, 1.0, 0.0, 1.0]]
    for ch in (0, 1, 31, 32, 63):
        s = torch.zeros(1, 64, device=gpu)
        s[0, ch] = 1
        w = pack_spikes(s)[0].cpu().numpy().view("<u8").item()
        assert w == 1 << ch
    with pytest.raises(ValueError, match="expected 4 words"):
        unpack_spikes(pack_spikes(torch.ones(1, 64, device=gpu)), 128)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 7, 33, 1000])
def test_pack_signed_zero_nan_and_row_counts(dtype, rows, gpu):
    """64-channel rows (the 16-byte-per-lane kernels): -0.0 packs as 0, NaN and
    tiny values as 1, for row counts that leave partial waves."""
    from spikeinfer_amd.kernels import pack_spikes, unpack_spikes

    g = torch.Generator().manual_seed(rows)
    vals = torch.tensor([0.0, -0.0, 1.0, -2.5, float("nan"), 1e-30, float("inf")], dtype=torch.float32)
    idx = torch.randint(0, len(vals), (rows, 128), generator=g)
    x = vals[idx].to(dtype)
    bits = (x.float() != 0) | x.float().isnan()
    words = pack_spikes(x.to(gpu))
    assert np.array_equal(words.cpu().numpy(), orc.np_pack(bits.numpy().astype(np.uint8)))
    assert torch.equal(unpack_spikes(words, 128, dtype).cpu(), bits.to(dtype))


def test_pack_noncontiguous(gpu):
    from spikeinfer_amd.kernels import pack_spikes, unpack_spikes

    spikes = (torch.rand(2, 4, 8, 64, device=gpu) > 0.5).float()
    view = spikes.permute(0, 2, 1, 3)
    assert torch.equal(unpack_spikes(pack_spikes(view), 64), view)


# ---- fused LIF + pack + cache write ---------------------------------------
@pytest.mark.parametrize("with_dense", [True, False])
@pytest.mark.parametrize("D", [64, 32, 128, 40])
@pytest.mark.parametrize("in_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_lif_pack_write_packed_buffer(D, in_dtype, with_dense, gpu):
    """Vectorised (16-byte, D % 64 == 0, no dense output) and scalar paths."""
    from spikeinfer_amd.kernels import lif_pack_write

    rng = np.random.default_rng(D)
    T, n_tok, H = 4, 37, 14
    beta, th = _rand_beta(rng, D), _rand_th(rng, D)
    # projection output [T, n_tok, H*D] viewed per head: no copy
    proj = torch.from_numpy(rng.standard_normal((T, n_tok, H * D)).astype(np.float32)).to(gpu)
    x = proj.to(in_dtype).view(T, n_tok, H, D)
    W = (D + 31) // 32
    out = torch.zeros((T, n_tok, H, W), dtype=torch.int32, device=gpu)
    dense = torch.empty((T, n_tok, H, D), dtype=in_dtype, device=gpu) if with_dense else None
    lif_pack_write(x, torch.from_numpy(beta).to(gpu), torch.from_numpy(th).to(gpu), out,
                   spikes_out=dense)
    want = np.zeros((T, n_tok, H, W), np.int32)
    orc.lif_pack_write(x.float().cpu().numpy(), beta, th, want)
    assert np.array_equal(out.cpu().numpy(), want)
    if with_dense:
        ws, _ = orc.lif(x.float().cpu().numpy(), beta, th)
        assert np.array_equal(dense.to(torch.uint8).cpu().numpy(), ws)


def test_lif_pack_write_cache_scatter(gpu):
    """Config-2 k/v site, reduced: random unique slots, bs=16, bf16 N(0,1)."""
    from spikeinfer_amd.kernels import lif_pack_write

    rng = np.random.default_rng(2)
    T, n_tok, H, D, S = 4, 512, 2, 64, 16 * 300
    x = torch.from_numpy(rng.standard_normal((T, n_tok, H, D)).astype(np.float32)).to(gpu).bfloat16()
    beta = np.full(D, 0.9, np.float32)
    th = np.full(D, 1.0, np.float32)
    slots = rng.permutation(S - 16)[:n_tok].astype(np.int64)
    slots[3] = -1       # skipped
    slots[4] = S + 5    # out of range: skipped, no fault
    cache = torch.full((T, H, S, 2), 123, dtype=torch.int32, device=gpu)
    lif_pack_write(x, torch.from_numpy(beta).to(gpu), torch.from_numpy(th).to(gpu), cache,
                   slot_mapping=torch.from_numpy(slots).to(gpu))
    want = np.full((T, H, S, 2), 123, np.int32)
    orc.lif_pack_write(x.float().cpu().numpy(), beta, th, want, slots)
    assert np.array_equal(cache.cpu().numpy(), want)


def test_lif_pack_write_matches_reference_composition(gpu):
    """Fused kernel == lif_multistep -> pack_spikes -> index_copy_ (attention.py:138-139)."""
    from spikeinfer_amd.kernels import lif_multistep, lif_pack_write, pack_spikes

    rng = np.random.default_rng(8)
    T, n_tok, H, D, S = 4, 64, 2, 64, 16 * 8
    x = torch.from_numpy(rng.standard_normal((T, n_tok, H, D)).astype(np.float32)).to(gpu).bfloat16()
    beta = torch.rand(D, device=gpu)
    th = torch.rand(D, device=gpu) * 0.5 + 0.1
    slots = torch.from_numpy(rng.permutation(S)[:n_tok].astype(np.int64)).to(gpu)
    fused = torch.zeros((T, H, S, 2), dtype=torch.int32, device=gpu)
    lif_pack_write(x, beta, th, fused, slot_mapping=slots)
    spk = lif_multistep(x.permute(0, 2, 1, 3), beta, th)  # [T, H, n_tok, D]
    comp = torch.zeros_like(fused)
    comp.index_copy_(2, slots, pack_spikes(spk))
    assert torch.equal(fused, comp)


@pytest.mark.parametrize("T", [4, 1, 3, 8])
@pytest.mark.parametrize("D", [64, 128, 32])
@pytest.mark.parametrize("in_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_lif_pack_write_sites_one_launch(D, in_dtype, T, gpu):
    """q (packed buffer, first n_dec tokens), k and v (cache scatter) with their
    own parameters in one spk_lif_pack_write_sites call: bit-exact against the
    oracle per site.  D = 32 and fp32 inputs take the per-site fallback; T = 1
    and 3 re-read the last timestep for the unused loads of the 4-step batch,
    T = 8 runs a second batch."""
    from spikeinfer_amd.kernels import lif_pack_write_sites

    rng = np.random.default_rng(300 + D + T)
    n_tok, n_dec, Hq, Hkv, S = 203, 150, 14, 2, 16 * 40
    W = (D + 31) // 32
    proj = rng.standard_normal((T, n_tok, (Hq + 2 * Hkv) * D)).astype(np.float32)
    x = torch.from_numpy(proj).to(gpu).to(in_dtype)
    xq = x[..., : Hq * D].view(T, n_tok, Hq, D)  # strided views of one projection output
    xk = x[..., Hq * D:(Hq + Hkv) * D].view(T, n_tok, Hkv, D)
    xv = x[..., (Hq + Hkv) * D:].view(T, n_tok, Hkv, D)
    params = [(_rand_beta(rng, D), _rand_th(rng, D)) for _ in range(3)]
    slots = rng.permutation(S)[:n_tok].astype(np.int64)
    slots[5] = -1  # pad token: skipped
    qbuf = torch.full((T, n_dec, Hq, W), 7, dtype=torch.int32, device=gpu)
    kc = torch.full((T, Hkv, S, W), 9, dtype=torch.int32, device=gpu)
    vc = torch.full_like(kc, 11)
    tp = [tuple(torch.from_numpy(a).to(gpu) for a in pr) for pr in params]
    lif_pack_write_sites([(xq[:, :n_dec], *tp[0], qbuf, False), (xk, *tp[1], kc, True),
                          (xv, *tp[2], vc, True)], torch.from_numpy(slots).to(gpu))
    want_q = np.full((T, n_dec, Hq, W), 7, np.int32)
    orc.lif_pack_write(xq[:, :n_dec].float().cpu().numpy(), *params[0], want_q)
    assert np.array_equal(qbuf.cpu().numpy(), want_q), "q"
    for xs, c, pr, fill, name in ((xk, kc, params[1], 9, "k"), (xv, vc, params[2], 11, "v")):
        want = np.full((T, Hkv, S, W), fill, np.int32)
        orc.lif_pack_write(xs.float().cpu().numpy(), *pr, want, slots)
        assert np.array_equal(c.cpu().numpy(), want), name


def test_lif_pack_write_sites_rejects_bad_arguments(gpu):
    from spikeinfer_amd.kernels import lif_pack_write_sites

    x = torch.zeros((4, 3, 2, 64), dtype=torch.bfloat16, device=gpu)
    b = torch.full((64,), 0.9, device=gpu)
    out = torch.zeros((4, 3, 2, 2), dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError, match="1 to 4"):
        lif_pack_write_sites([])
    with pytest.raises(ValueError, match="slot_mapping"):
        lif_pack_write_sites([(x, b, b, out, True)])
    with pytest.raises(ValueError, match="same x dtype"):
        lif_pack_write_sites([(x, b, b, out, False), (x.half(), b, b, out, False)])


@pytest.mark.parametrize("in_dtype", [torch.bfloat16, torch.float16])
def test_lif_gate_vector_path(in_dtype, gpu):
    """Config-2 MLP-gate shape, reduced: [T, tokens, 4864] half-precision in and
    out (16-byte vector path), beta 0.9, threshold 1.0."""
    from spikeinfer_amd.kernels import lif_multistep

    rng = np.random.default_rng(2)
    x = torch.from_numpy(rng.standard_normal((4, 96, 4864)).astype(np.float32)).to(gpu).to(in_dtype)
    beta = torch.full((4864,), 0.9, device=gpu)
    th = torch.full((4864,), 1.0, device=gpu)
    s, u = lif_multistep(x, beta, th, return_membrane=True)
    assert s.dtype == in_dtype
    ws, wu = orc.lif(x.float().cpu().numpy(), beta.cpu().numpy(), th.cpu().numpy())
    assert np.array_equal(s.float().cpu().numpy().astype(np.uint8), ws)
    assert np.array_equal(u.cpu().numpy(), wu)
