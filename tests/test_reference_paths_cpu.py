"""The package's eager-torch restatements of the reference's non-kernel paths
(lif_multistep_ref, paged_spike_attn_decode_ref, paged_spike_attn_decode_cpu)
against the C oracle, on the CPU; and the reference's full kernel export list
(spikeinfer/kernels/__init__.py:1-29) importable from spikeinfer_amd.kernels."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import attn_case, oracle_attn
from oracle import oracle as orc

REFERENCE_KERNEL_NAMES = [
    "lif_multistep", "lif_multistep_ref", "validate_thresholds", "pack_spikes",
    "unpack_spikes", "packed_width", "packed_bytes_per_token", "BITS_PER_WORD",
    "paged_spike_attn_decode", "paged_spike_attn_decode_ref", "paged_spike_attn_decode_cpu",
    "gather_kv_unpacked",
]


def test_every_reference_kernel_name_is_exported():
    import spikeinfer_amd.kernels as k

    missing = [n for n in REFERENCE_KERNEL_NAMES if not hasattr(k, n)]
    assert not missing, missing
    assert set(REFERENCE_KERNEL_NAMES) <= set(k.__all__)


def _t(case):
    return dict(q_packed=torch.from_numpy(case["q"]), k_cache=torch.from_numpy(case["k"]),
                v_cache=torch.from_numpy(case["v"]), block_tables=torch.from_numpy(case["tables"]),
                seq_lens=torch.from_numpy(case["lens"]), head_dim=case["head_dim"],
                block_size=case["block_size"], num_q_heads=case["num_q_heads"],
                num_kv_heads=case["num_kv_heads"])


@pytest.mark.parametrize("fn_name", ["paged_spike_attn_decode_ref", "paged_spike_attn_decode_cpu"])
@pytest.mark.parametrize("lens,bs,hq,hkv,hd", [
    ([1], 16, 14, 2, 64), ([7, 33, 128], 16, 14, 2, 64), ([1, 5, 40, 97], 32, 4, 4, 64),
    ([64] * 8, 16, 8, 1, 64), ([10, 50], 16, 4, 2, 40), ([300, 129], 16, 6, 2, 128),
])
def test_eager_attention_paths_match_oracle(fn_name, lens, bs, hq, hkv, hd):
    import spikeinfer_amd.kernels as k

    case = attn_case(lens, block_size=bs, q_heads=hq, kv_heads=hkv, head_dim=hd, seed=len(lens) + bs)
    got = getattr(k, fn_name)(**_t(case)).numpy().astype(np.float64)
    np.testing.assert_allclose(got, oracle_attn(case), atol=1e-5, rtol=0)


def test_cpu_path_groups_under_a_small_budget(monkeypatch):
    """A tiny gather budget splits the batch into many runs (each at least one
    sequence); the ragged runs take the -inf mask.  Same result."""
    from spikeinfer_amd.kernels import paged_spike_attn_decode_cpu

    monkeypatch.setenv("SPIKEINFER_CPU_GATHER_BUDGET_MB", "0.05")
    case = attn_case([5, 300, 17, 17, 1, 200, 64], block_size=16, seed=3)
    got = paged_spike_attn_decode_cpu(**_t(case)).numpy().astype(np.float64)
    np.testing.assert_allclose(got, oracle_attn(case), atol=1e-5, rtol=0)


def test_cpu_path_bf16_out():
    from spikeinfer_amd.kernels import paged_spike_attn_decode_cpu

    case = attn_case([40, 41], seed=9)
    got = paged_spike_attn_decode_cpu(**_t(case), dtype=torch.bfloat16)
    assert got.dtype == torch.bfloat16
    want = torch.from_numpy(oracle_attn(case)).float()
    assert ((got.float() - want).abs() <= want.abs() * 2.0 ** -8 + 1e-6).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lif_multistep_ref_matches_oracle_bit_exactly(dtype):
    from spikeinfer_amd.kernels import lif_multistep_ref

    g = torch.Generator().manual_seed(4)
    x = (torch.randn(6, 40, 96, generator=g) * 1.5).to(dtype)
    beta = torch.rand(96, generator=g) * 1.4 - 0.2  # exercises the clamp
    th = torch.rand(96, generator=g) + 0.5
    s, u = lif_multistep_ref(x, beta, th)
    s_o, u_o = orc.lif(x.float().numpy(), beta.numpy(), th.numpy())
    assert np.array_equal(s.float().numpy(), s_o.astype(np.float32))
    assert np.array_equal(u.numpy(), u_o)
    assert s.dtype == dtype


def test_lif_multistep_ref_hand_case():
    """beta 0.9, threshold 1, I = 1: u0 = 1.0 sits exactly on the threshold, so
    t = 0 does not fire; spikes [0, 1, 1, 1]."""
    from spikeinfer_amd.kernels import lif_multistep_ref

    s, _ = lif_multistep_ref(torch.ones(4, 1, 1), torch.tensor([0.9]), torch.tensor([1.0]))
    assert s.flatten().tolist() == [0.0, 1.0, 1.0, 1.0]


def test_unpack_spikes_torch_matches_packbits():
    from spikeinfer_amd.kernels import unpack_spikes_torch

    rng = np.random.default_rng(1)
    bits = (rng.random((5, 3, 70)) < 0.3).astype(np.uint8)
    words = orc.np_pack(bits)
    got = unpack_spikes_torch(torch.from_numpy(words), 70, torch.uint8).numpy()
    assert np.array_equal(got, bits)
    with pytest.raises(ValueError, match="words"):
        unpack_spikes_torch(torch.from_numpy(words), 100)


@pytest.mark.parametrize("channels", [1, 31, 32, 33, 64, 128, 4864])
def test_pack_spikes_torch_matches_packbits(channels):
    """The reference's CPU packing restated: equal to the numpy packbits twin,
    any nonzero (negative, NaN) packs as 1, all-ones words wrap to -1."""
    from spikeinfer_amd.kernels import pack_spikes_torch

    rng = np.random.default_rng(channels)
    bits = (rng.random((3, 5, channels)) < 0.3).astype(np.uint8)
    x = torch.from_numpy(bits.astype(np.float32))
    x[x != 0] = torch.tensor([-2.0, float("nan"), 0.5]).repeat(int((x != 0).sum()) // 3 + 1)[: int((x != 0).sum())]
    got = pack_spikes_torch(x).numpy()
    assert got.dtype == np.int32
    assert np.array_equal(got, orc.np_pack(bits))
    ones = pack_spikes_torch(torch.ones(2, 64))
    assert (ones == -1).all()


def test_reference_cpu_lif_pack_write_matches_oracle():
    """The torch CPU form of the k/v cache write the bench times
    (lif_multistep_ref -> pack_spikes_torch -> index_copy_, attention.py:138-139)
    writes the same cache bytes as the C oracle's fused restatement."""
    from spikeinfer_amd.kernels import lif_multistep_ref, pack_spikes_torch

    rng = np.random.default_rng(4)
    T, n_tok, H, D, S = 4, 50, 2, 64, 16 * 8
    x = torch.from_numpy(rng.standard_normal((T, n_tok, H, D)).astype(np.float32)).bfloat16()
    beta = torch.from_numpy((rng.random(D) * 1.2).astype(np.float32))
    th = torch.from_numpy((rng.random(D) * 0.9 + 0.1).astype(np.float32))
    slots = torch.from_numpy(rng.permutation(S)[:n_tok].astype(np.int64))
    cache = torch.zeros((T, H, S, 2), dtype=torch.int32)
    words = pack_spikes_torch(lif_multistep_ref(x, beta, th)[0])
    cache.index_copy_(2, slots, words.permute(0, 2, 1, 3))
    want = np.zeros((T, H, S, 2), np.int32)
    orc.lif_pack_write(x.float().numpy(), beta.numpy(), th.numpy(), want, slots.numpy())
    assert np.array_equal(cache.numpy(), want)
