"""Every output element of the decode-step kernels is written, at ragged
sizes: each op runs once into a NaN-filled ``out`` and once into a zero-filled
one, and the two results must be identical and finite (an element a kernel
skips keeps its fill value, so the two runs would differ there).  Shapes:
row counts that are not multiples of the kernels' 16- and 64-row groups,
column counts with a partial last column range, and the config-5 widths."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _twice(fn, shape, dtype, gpu):
    outs = []
    for fill in (float("nan"), 0.0):
        out = torch.full(shape, fill, dtype=dtype, device=gpu)
        fn(out)
        torch.cuda.synchronize()
        outs.append(out)
    a, b = outs
    assert bool(torch.isfinite(a.float()).all()), "an element kept its NaN fill"
    assert torch.equal(a, b)
    return a


@pytest.mark.parametrize("M,N,K,bias", [(1, 1152, 896, True), (37, 896, 896, False), (148, 1152, 896, True),
                                        (256, 896, 896, False), (5, 20480, 640, False),
                                        (4, 896, 4864, False), (99, 896, 4864, False),
                                        (64, 151936, 896, False), (3, 48, 128, True)])
def test_linear_decode_writes_every_element(M, N, K, bias, gpu):
    from spikeinfer_amd.kernels.decoder_ops import linear_decode, pack_linear

    print(f"outputs written: linear_decode M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(M + N)
    x = torch.randn((M, K), generator=g, device=gpu).bfloat16()
    w = (torch.randn((N, K), generator=g, device=gpu) * 0.05).bfloat16()
    b = (torch.randn(N, generator=g, device=gpu) * 0.1).bfloat16() if bias else None
    wp = pack_linear(w)
    ran = []
    _twice(lambda out: ran.append(linear_decode(x, wp, b, out=out) is not None), (M, N), torch.bfloat16, gpu)
    assert all(ran), "shape outside the kernel's range"


@pytest.mark.parametrize("T,n", [(4, 64), (4, 37), (1, 5), (3, 16), (4, 1)])
def test_mlp_gate_lif_writes_every_element(T, n, gpu):
    from spikeinfer_amd.kernels.decoder_ops import mlp_gate_lif, pack_gate_up

    H, I = 896, 4864
    print(f"outputs written: mlp_gate_lif T={T} n={n}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(T * 100 + n)
    x = torch.randn((T, n, H), generator=g, device=gpu).bfloat16()
    w = (torch.randn((2 * I, H), generator=g, device=gpu) * 0.05).bfloat16()
    beta = 0.6 + 0.4 * torch.rand(I, generator=g, device=gpu)
    th = 0.5 + torch.rand(I, generator=g, device=gpu)
    wp = pack_gate_up(w)
    ran = []
    _twice(lambda out: ran.append(mlp_gate_lif(x, wp, beta, th, out=out) is not None), (T, n, I),
           torch.bfloat16, gpu)
    assert all(ran), "shape outside the kernel's range"


@pytest.mark.parametrize("rows,hidden", [(1, 896), (37 * 4, 896), (256, 896), (7, 2056)])
def test_add_rmsnorm_writes_every_element(rows, hidden, gpu):
    from spikeinfer_amd.kernels.decoder_ops import add_rmsnorm

    print(f"outputs written: add_rmsnorm rows={rows} hidden={hidden}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(rows + hidden)
    h0 = torch.randn((rows, hidden), generator=g, device=gpu).bfloat16()
    d = torch.randn((rows, hidden), generator=g, device=gpu).bfloat16()
    w = (1 + 0.1 * torch.randn(hidden, generator=g, device=gpu)).bfloat16()
    _twice(lambda out: add_rmsnorm(h0.clone(), d, w, 1e-6, out=out), (rows, hidden), torch.bfloat16, gpu)


@pytest.mark.parametrize("T,rows,I", [(4, 37, 4864), (1, 3, 64), (4, 64, 4864)])
def test_lif_gate_mul_writes_every_element(T, rows, I, gpu):
    from spikeinfer_amd.kernels.decoder_ops import lif_gate_mul

    print(f"outputs written: lif_gate_mul T={T} rows={rows} I={I}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(T + rows + I)
    gu = (torch.randn((T, rows, 2 * I), generator=g, device=gpu) * 1.5).bfloat16()
    beta = 0.6 + 0.4 * torch.rand(I, generator=g, device=gpu)
    th = 0.5 + torch.rand(I, generator=g, device=gpu)
    _twice(lambda out: lif_gate_mul(gu, beta, th, out=out), (T, rows, I), torch.bfloat16, gpu)
