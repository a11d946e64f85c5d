"""Split-context operators (partials + combine), the one-launch prefill
gather-unpack, sequence lengths past the block table, and mixed-dtype LIF
parameters -- through the C-ABI against the CPU oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import attn_case, oracle_attn
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _dev(case, gpu):
    return dict(
        q_packed=torch.from_numpy(case["q"]).to(gpu), k_cache=torch.from_numpy(case["k"]).to(gpu),
        v_cache=torch.from_numpy(case["v"]).to(gpu),
        block_tables=torch.from_numpy(case["tables"]).to(gpu),
        seq_lens=torch.from_numpy(case["lens"]).to(gpu), head_dim=case["head_dim"],
        block_size=case["block_size"], num_q_heads=case["num_q_heads"],
        num_kv_heads=case["num_kv_heads"])


def _close(got, want, ctx):
    got = got.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - want).max()
    assert err <= 1e-3 and err / max(np.abs(want).max(), 1e-6) < 1e-5, f"{ctx}: err {err:.2e}"


@pytest.fixture(params=["auto", "general"])
def path(request, monkeypatch):
    monkeypatch.setenv("SPIKEINFER_AMD_ATTN_PATH", request.param)
    return request.param


# ---- partials + combine ------------------------------------------------------
@pytest.mark.parametrize("part_len", [16, 256, 1024, 4096, 32768])
@pytest.mark.parametrize("lens,hd", [([1, 0, 300, 5000, 17], 64), ([9000, 40, 129], 64),
                                     ([700, 0, 2100], 128)])
def test_partials_then_combine_match_oracle(part_len, lens, hd, path, gpu):
    from spikeinfer_amd.kernels import combine_partitions, paged_spike_attn_decode_partials

    case = attn_case(lens, block_size=16, T=2, head_dim=hd, density=0.2, q_density=0.2,
                     seed=part_len + len(lens))
    print(f"partials part_len={part_len} lens={lens} hd={hd} path={path}", flush=True)
    d = _dev(case, gpu)
    parts = paged_spike_attn_decode_partials(**d, part_len=part_len)
    out = combine_partitions(parts, d["seq_lens"], part_len)
    torch.cuda.synchronize()
    _close(out, oracle_attn(case), f"part_len={part_len}")
    P = parts.shape[0]
    assert P == -(-case["tables"].shape[1] * 16 // part_len)


def test_partials_of_different_splits_add(gpu):
    """With the fixed softmax offset popcount(q), the partials of two
    adjacent partitions of length L sum to the partial of the 2L partition
    (up to fp32 summation order)."""
    from spikeinfer_amd.kernels import paged_spike_attn_decode_partials

    case = attn_case([4096, 3000, 2048], block_size=16, T=1, density=0.3, q_density=0.3, seed=3)
    d = _dev(case, gpu)
    a = paged_spike_attn_decode_partials(**d, part_len=512)
    b = paged_spike_attn_decode_partials(**d, part_len=1024)
    torch.cuda.synchronize()
    for n, L in enumerate(case["lens"]):
        for p in range(-(-int(L) // 1024)):
            lo = a[2 * p, :, n]
            hi = a[2 * p + 1, :, n] if (2 * p + 1) * 512 < L else torch.zeros_like(lo)
            torch.testing.assert_close(lo + hi, b[p, :, n], rtol=2e-6, atol=1e-6)


def test_combine_of_a_split_across_launches(gpu):
    """A context split between two callers (e.g. two devices, each holding
    half of the blocks): each computes partials over its half, zero-padded
    partition axes are stacked, and one combine gives the full attention."""
    from spikeinfer_amd.kernels import combine_partitions, paged_spike_attn_decode_partials

    L, bs, pl = 2048, 16, 1024
    case = attn_case([L, L], block_size=bs, T=2, density=0.2, q_density=0.25, seed=8)
    d = _dev(case, gpu)
    full = paged_spike_attn_decode_partials(**d, part_len=pl)
    # second half only: table shifted by the first half's blocks, lengths L/2
    d2 = dict(d, block_tables=d["block_tables"][:, pl // bs:].contiguous(),
              seq_lens=torch.full_like(d["seq_lens"], L - pl))
    half2 = paged_spike_attn_decode_partials(**d2, part_len=pl)
    stacked = torch.stack([full[0], half2[0]])
    out = combine_partitions(stacked, d["seq_lens"], pl)
    torch.cuda.synchronize()
    _close(out, oracle_attn(case), "cross-launch split")


def test_partials_rejects_bad_part_len(gpu):
    from spikeinfer_amd.kernels import paged_spike_attn_decode_partials

    d = _dev(attn_case([40]), gpu)
    for bad in (24, 0, 65536):
        with pytest.raises(ValueError, match="part_len"):
            paged_spike_attn_decode_partials(**d, part_len=bad)


# ---- lengths past the block table --------------------------------------------
@pytest.mark.parametrize("lens", [[100, 2000], [40000, 5], [9000, 300]])
def test_seq_len_past_the_table_is_clamped(lens, path, gpu):
    """seq_len beyond max_blocks * block_size: the kernels read only what the
    table addresses (the result equals the clamped length's), on every path,
    split or not."""
    from spikeinfer_amd.kernels import paged_spike_attn_decode

    table_len = [min(x, 1024) for x in lens]
    case = attn_case(table_len, block_size=16, T=2, density=0.2, q_density=0.2, seed=sum(lens))
    want = oracle_attn(case)
    d = _dev(case, gpu)
    d["seq_lens"] = torch.tensor(lens, dtype=torch.int32, device=gpu)
    # tables only as wide as the clamped lengths need
    got = paged_spike_attn_decode(**d)
    torch.cuda.synchronize()
    cap = case["tables"].shape[1] * 16
    assert [min(x, cap) for x in lens] == table_len
    _close(got, want, f"lens={lens}")


# ---- prefill gather-unpack ---------------------------------------------------
def _slots(table, seq_len, bs):
    p = np.arange(seq_len)
    return table[p // bs].astype(np.int64) * bs + p % bs


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.uint8,
                                   torch.bool, torch.int32])
@pytest.mark.parametrize("hd,seq_len,bs", [(64, 300, 16), (128, 33, 32), (40, 70, 16), (64, 1, 8)])
def test_gather_unpack_matches_slot_gather(dtype, hd, seq_len, bs, gpu):
    from spikeinfer_amd.kernels import gather_kv_unpacked, gather_kv_unpacked_pair

    case = attn_case([seq_len, 50], block_size=bs, head_dim=hd, T=3, density=0.3, seed=hd + seq_len)
    table = case["tables"][0]
    slots = _slots(table, seq_len, bs)
    want_k = orc.unpack(case["k"][:, :, slots], hd)  # [T, H, S, D] uint8
    want_v = orc.unpack(case["v"][:, :, slots], hd)
    d = _dev(case, gpu)
    k, v = gather_kv_unpacked_pair(d["k_cache"], d["v_cache"], d["block_tables"][0], seq_len, hd,
                                   bs, dtype)
    k1 = gather_kv_unpacked(d["k_cache"], d["block_tables"][0], seq_len, hd, bs, dtype)
    torch.cuda.synchronize()
    assert k.dtype == dtype and tuple(k.shape) == want_k.shape
    assert np.array_equal(k.cpu().to(torch.uint8).numpy(), want_k)
    assert np.array_equal(v.cpu().to(torch.uint8).numpy(), want_v)
    assert torch.equal(k1, k)


def test_gather_unpack_past_table_and_outside_cache_read_zero(gpu):
    from spikeinfer_amd.kernels import gather_kv_unpacked

    case = attn_case([64], block_size=16, seed=2, density=0.5)
    d = _dev(case, gpu)
    table = d["block_tables"][0].clone()  # 4 entries
    table[1] = 10 ** 6                    # outside the cache
    got = gather_kv_unpacked(d["k_cache"], table, 80, 64, 16, torch.float32).cpu()
    assert got[:, :, 16:32].abs().sum() == 0 and got[:, :, 64:].abs().sum() == 0
    slots = _slots(case["tables"][0], 16, 16)
    assert np.array_equal(got[:, :, :16].to(torch.uint8).numpy(), orc.unpack(case["k"][:, :, slots], 64))


# ---- mixed LIF parameter dtypes ------------------------------------------------
def test_lif_mixed_param_dtypes_use_each_in_its_own_precision(gpu):
    """bf16 beta with an fp32 threshold that bf16 cannot hold: the threshold
    must not be rounded to bf16 (the reference upcasts each parameter)."""
    from spikeinfer_amd.kernels import lif_multistep, lif_pack_write

    T, M, N = 4, 512, 64
    th32 = np.float32(1.0 + 2.0 ** -12)  # rounds to 1.0 in bf16
    rng = np.random.default_rng(5)
    # currents straddling the true threshold: u after one step = x
    x = np.full((T, M, N), th32, np.float32)
    x[0] = th32 + (rng.integers(-2, 3, (M, N)) * 2.0 ** -14).astype(np.float32)
    beta_bf = torch.full((N,), 0.9, dtype=torch.bfloat16)
    th = np.full(N, th32, np.float32)
    want_s, _ = orc.lif(x, beta_bf.float().numpy(), th)
    got = lif_multistep(torch.from_numpy(x).to(gpu), beta_bf.to(gpu), torch.from_numpy(th).to(gpu))
    assert np.array_equal(got.cpu().numpy().astype(np.uint8), want_s)
    buf = torch.zeros((T, M, 1, 2), dtype=torch.int32, device=gpu)
    lif_pack_write(torch.from_numpy(x).to(gpu).view(T, M, 1, N), beta_bf.to(gpu),
                   torch.from_numpy(th).to(gpu), buf)
    assert np.array_equal(buf.cpu().numpy().reshape(T, M, 2), orc.pack(want_s))
