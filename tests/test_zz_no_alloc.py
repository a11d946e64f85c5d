"""spk_decode_attn_noalloc (the allocation-free decode attention entry point)
through the C-ABI against spk_decode_attn with a caller workspace: identical
outputs on two calls in a row, the second with a smaller input, both needing
scratch (the launch-order list, then the partial sums of a context longer
than one partition); and a
shape whose scratch exceeds the fixed size is rejected."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cases import attn_case

pytestmark = pytest.mark.gpu


def _noalloc(lib, d, out):
    from spikeinfer_amd import _lib

    q, k, v, bt, lens = d["q_packed"], d["k_cache"], d["v_cache"], d["block_tables"], d["seq_lens"]
    T, N, Hq, _ = q.shape
    return lib.spk_decode_attn_noalloc(
        q.data_ptr(), _lib.strides(q), k.data_ptr(), _lib.strides(k), v.data_ptr(), _lib.strides(v),
        k.shape[2], bt.data_ptr(), bt.stride(0), bt.stride(1), lens.data_ptr(), out.data_ptr(),
        _lib.dtype_code(out.dtype), _lib.strides(out), T, N, Hq, d["num_kv_heads"], d["head_dim"],
        d["block_size"], bt.shape[1], 1.0 / math.sqrt(d["head_dim"]), _lib.stream_of(q.device))


def _dev(case, gpu):
    return dict(q_packed=torch.from_numpy(case["q"]).to(gpu), k_cache=torch.from_numpy(case["k"]).to(gpu),
                v_cache=torch.from_numpy(case["v"]).to(gpu),
                block_tables=torch.from_numpy(case["tables"]).to(gpu),
                seq_lens=torch.from_numpy(case["lens"]).to(gpu), head_dim=case["head_dim"],
                block_size=case["block_size"], num_q_heads=case["num_q_heads"],
                num_kv_heads=case["num_kv_heads"])


def _ragged(n, seed, longest):
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, 200, n)
    lens[rng.choice(n, 20, replace=False)] = 0
    lens[rng.choice(n, 3, replace=False)] = [longest, 12000, 8193]
    return attn_case(lens.tolist(), block_size=16, T=1, density=0.2, q_density=0.2, seed=seed,
                     compact=True)


def test_noalloc_matches_workspace_entry_on_consecutive_calls(gpu, monkeypatch):
    from spikeinfer_amd import _lib
    from spikeinfer_amd.kernels import decode_attn_workspace_bytes, paged_spike_attn_decode

    monkeypatch.delenv("SPIKEINFER_AMD_ATTN_PATH", raising=False)
    lib = _lib.load()
    # launch-order list in scratch, then the partial sums of a context past
    # one 32768-token partition
    for n, longest in ((4100, 8200), (300, 40000)):
        case = _ragged(n, n, longest)
        d = _dev(case, gpu)
        need = decode_attn_workspace_bytes(1, n, 14, 2, 64, 16, case["tables"].shape[1])
        assert 0 < need <= _lib.DECODE_ATTN_SCRATCH_BYTES
        print(f"noalloc n={n} scratch={need}", flush=True)
        want = paged_spike_attn_decode(**d)
        got = torch.full_like(want, float("nan"))
        assert _noalloc(lib, d, got) == 0, lib.spk_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"n={n}: noalloc output differs"


def test_noalloc_rejects_scratch_beyond_its_size(gpu):
    from spikeinfer_amd import _lib

    lib = _lib.load()
    T, N, Hq, Hkv, hd, bs, max_blocks = 8, 32, 64, 4, 128, 16, 65536
    from spikeinfer_amd.kernels import decode_attn_workspace_bytes

    assert decode_attn_workspace_bytes(T, N, Hq, Hkv, hd, bs, max_blocks) > _lib.DECODE_ATTN_SCRATCH_BYTES
    d = dict(q_packed=torch.zeros((T, N, Hq, 4), dtype=torch.int32, device=gpu),
             k_cache=torch.zeros((T, Hkv, 16, 4), dtype=torch.int32, device=gpu),
             v_cache=torch.zeros((T, Hkv, 16, 4), dtype=torch.int32, device=gpu),
             block_tables=torch.zeros((N, max_blocks), dtype=torch.int32, device=gpu),
             seq_lens=torch.ones(N, dtype=torch.int32, device=gpu), head_dim=hd, block_size=bs,
             num_kv_heads=Hkv)
    out = torch.empty((T, N, Hq, hd), device=gpu)
    assert _noalloc(lib, d, out) == _lib.SPK_EINVAL
    assert b"scratch" in lib.spk_last_error()
