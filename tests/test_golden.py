"""Committed golden fixtures (tests/golden/, written by make_golden.py from the
numpy / pure-Python twins) checked against the C oracle on the CPU and against
the HIP kernels, through the C-ABI, on the GPU."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
D, BS, HQ, HKV = 64, 16, 14, 2


def _npz(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _hand():
    with open(os.path.join(GOLDEN, "hand_cases.json")) as f:
        return json.load(f)


# ---- CPU: the C oracle reproduces the fixtures ------------------------------
def test_oracle_config1_attention():
    g = _npz("config1_attn.npz")
    out = orc.decode_attn(g["q"], g["k"], g["v"], g["tables"], g["lens"], D, BS, HQ, HKV)
    np.testing.assert_allclose(out, g["out"], rtol=0, atol=1e-12)
    sc = orc.decode_scores(g["q"], g["k"], g["tables"], g["lens"], D, BS, HQ, HKV, 128)
    assert np.array_equal(sc, g["scores"])


def test_oracle_lif_boundary():
    g = _npz("lif_boundary.npz")
    s, u = orc.lif(g["x"], g["beta"], g["thr"])
    assert np.array_equal(np.packbits(s, axis=-1, bitorder="little"), g["spikes_packed"])
    assert np.array_equal(u, g["u"])


def test_oracle_hand_cases():
    h = _hand()
    for name in ("pack_all_ones", "pack_c33_tail"):
        c = h[name]
        assert orc.pack(np.ones((1, c["channels"]), np.uint8))[0].tolist() == c["words"]
    c = h["pack_single_channel"]
    for ch, w in zip(c["set"], c["words"]):
        b = np.zeros((1, 64), np.uint8)
        b[0, ch] = 1
        assert orc.pack(b)[0].tolist() == w
    c = h["lif_constant_current"]
    s, _ = orc.lif(np.full((c["T"], 1, 1), c["current"], np.float32),
                   np.array([c["beta"]], np.float32), np.array([c["threshold"]], np.float32))
    assert s[:, 0, 0].tolist() == c["spikes"]


def test_host_conventions_hand_cases():
    from spikeinfer_amd.kernels import packed_bytes_per_token
    from spikeinfer_amd.spike_cache import slot_mapping

    h = _hand()
    c = h["slot_matrix"]
    assert [slot_mapping(t, 0, c["len"], c["block_size"]) for t in c["tables"]] == c["slots"]
    c = h["bytes_per_token"]
    assert packed_bytes_per_token(c["layers"], c["T"], c["kv_heads"], c["head_dim"]) == c["bytes"]


# ---- GPU: the HIP kernels reproduce the fixtures ----------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("path", ["auto", "general"])
def test_gpu_config1_attention(gpu, path, monkeypatch):
    import torch

    from spikeinfer_amd.kernels import paged_spike_attn_decode, paged_spike_attn_scores

    if path == "general":
        monkeypatch.setenv("SPIKEINFER_AMD_ATTN_PATH", "general")
    g = _npz("config1_attn.npz")
    t = {k: torch.from_numpy(g[k]).to(gpu) for k in ("q", "k", "v", "tables", "lens")}
    out = paged_spike_attn_decode(t["q"], t["k"], t["v"], t["tables"], t["lens"], head_dim=D,
                                  block_size=BS, num_q_heads=HQ, num_kv_heads=HKV)
    sc = paged_spike_attn_scores(t["q"], t["k"], t["tables"], t["lens"], D, BS, HQ, HKV, 128)
    assert np.array_equal(sc.cpu().numpy(), g["scores"])
    assert np.abs(out.cpu().numpy() - g["out"]).max() <= 1e-3


@pytest.mark.gpu
def test_gpu_lif_boundary(gpu):
    import torch

    from spikeinfer_amd.kernels import lif_multistep

    g = _npz("lif_boundary.npz")
    x = torch.from_numpy(g["x"]).to(gpu)
    s, u = lif_multistep(x, torch.from_numpy(g["beta"]).to(gpu), torch.from_numpy(g["thr"]).to(gpu),
                         return_membrane=True)
    bits = (s.cpu().numpy() != 0).astype(np.uint8)
    assert np.array_equal(np.packbits(bits, axis=-1, bitorder="little"), g["spikes_packed"])
    assert np.array_equal(u.cpu().numpy(), g["u"])


@pytest.mark.gpu
def test_gpu_pack_hand_cases(gpu):
    import torch

    from spikeinfer_amd.kernels import pack_spikes

    h = _hand()
    for name in ("pack_all_ones", "pack_c33_tail"):
        c = h[name]
        assert pack_spikes(torch.ones((1, c["channels"]), device=gpu))[0].tolist() == c["words"]
    c = h["pack_single_channel"]
    for ch, w in zip(c["set"], c["words"]):
        b = torch.zeros((1, 64), device=gpu)
        b[0, ch] = 1
        assert pack_spikes(b)[0].tolist() == w
