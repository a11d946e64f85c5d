"""The test-only torch restatement of the reference forward (tests/model_ref.py)
pinned on the CPU: its LIF recurrence and bit packing against the oracle's
independent numpy twins (np_lif: float32, one rounding per operation;
np_pack / np_unpack: numpy packbits), bit for bit, including the channel
counts that leave a partial last word and timestep-broadcast parameters."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from model_ref import lif_ref, pack_ref, unpack_ref
from oracle import oracle as orc


@pytest.mark.parametrize("T,C,dtype", [(4, 64, torch.float32), (4, 896, torch.bfloat16), (1, 37, torch.float16),
                                       (8, 128, torch.bfloat16)])
def test_lif_ref_matches_np_lif(T, C, dtype):
    g = torch.Generator().manual_seed(T * 1000 + C)
    x = (torch.randn((T, 5, C), generator=g) * 1.5 + 0.3).to(dtype)
    beta = (torch.rand(C, generator=g) * 1.4 - 0.2).to(dtype)  # values outside [0, 1] are clamped
    th = (0.5 + torch.rand(C, generator=g)).to(dtype)
    got = lif_ref(x, beta, th)
    want, _ = orc.np_lif(x.float().numpy(), beta.float().numpy(), th.float().numpy())
    assert got.dtype == dtype
    np.testing.assert_array_equal(got.float().numpy().astype(np.uint8), want)


@pytest.mark.parametrize("C", [1, 31, 32, 33, 64, 100, 128])
def test_pack_ref_and_unpack_ref_match_numpy_twins(C):
    rng = np.random.default_rng(C)
    bits = (rng.random((3, 7, C)) < 0.3).astype(np.uint8)
    got = pack_ref(torch.from_numpy(bits.astype(np.float32)))
    np.testing.assert_array_equal(got.numpy(), orc.np_pack(bits))
    back = unpack_ref(got, C, torch.float32)
    np.testing.assert_array_equal(back.numpy().astype(np.uint8), orc.np_unpack(got.numpy(), C))
    np.testing.assert_array_equal(back.numpy().astype(np.uint8), bits)
