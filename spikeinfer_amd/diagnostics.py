"""Kernel self-check: runs the HIP kernels on small inputs and compares them
with the reference's own eager paths, as the reference's doctor does for its
Triton kernels (spikeinfer/diagnostics.py:289-333: the packing round trip and
the LIF kernel against ``lif_multistep_ref``, "actually compile and run the
kernels, rather than trusting the imports").  Here the checks also cover the
paged decode attention against the reference's CPU strategy, within the
1e-3 max-abs the attention output is held to.

The eager paths used as the yardstick are the package's restatements in
``kernels/reference_paths.py`` (which the operators never call).  On a host
without a GPU the kernel checks report ``skip``: the HIP library runs only on
an MI355X (gfx950).

    python -m spikeinfer_amd.diagnostics      # prints the report; exit 1 on a failure
"""
from __future__ import annotations

import sys
from dataclasses import dataclass, field

import torch

from . import _lib


@dataclass
class Check:
    name: str
    status: str  # "ok", "fail" or "skip"
    detail: str
    data: dict = field(default_factory=dict)


def _library() -> Check:
    try:
        lib = _lib.load()
    except Exception as exc:  # missing or stale build
        return Check("library", "fail", f"{type(exc).__name__}: {exc}")
    return Check("library", "ok", f"{_lib.LIB_PATH} (ABI {lib.spk_abi_version()}, "
                                  f"{len(_lib.EXPORTED_SYMBOLS)} entry points)",
                 {"abi": int(lib.spk_abi_version())})


def _packing(dev: torch.device) -> Check:
    from .kernels import pack_spikes, unpack_spikes

    g = torch.Generator(device=dev).manual_seed(1)
    spikes = (torch.rand((4, 8, 96), generator=g, device=dev) < 0.5).float()
    back = unpack_spikes(pack_spikes(spikes), 96, torch.float32)
    torch.cuda.synchronize(dev)
    if torch.equal(back, spikes):
        return Check("packing round trip", "ok", "exact (C = 96: two words, one partial)")
    return Check("packing round trip", "fail", "unpack(pack(x)) is not x")


def _lif(dev: torch.device) -> Check:
    from .kernels import lif_multistep, lif_multistep_ref

    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn((4, 64, 32), generator=g, device=dev) * 1.5
    beta = 0.5 + 0.5 * torch.rand(32, generator=g, device=dev)
    th = 0.5 + torch.rand(32, generator=g, device=dev)
    got = lif_multistep(x, beta, th)
    want, _ = lif_multistep_ref(x, beta, th)
    torch.cuda.synchronize(dev)
    ok = torch.equal(got, want)
    return Check("lif kernel", "ok" if ok else "fail",
                 "bit-exact against lif_multistep_ref" if ok else
                 f"{int((got != want).sum())} spikes differ from lif_multistep_ref",
                 {"exact": ok})


def _attention(dev: torch.device) -> Check:
    from .kernels import paged_spike_attn_decode, paged_spike_attn_decode_cpu

    T, N, Hq, Hkv, D, bs, nblk = 2, 5, 14, 2, 64, 16, 40
    g = torch.Generator(device=dev).manual_seed(3)
    k = torch.randint(-2**31, 2**31 - 1, (T, Hkv, nblk * bs, D // 32), generator=g, device=dev,
                      dtype=torch.int32)
    v = torch.randint(-2**31, 2**31 - 1, (T, Hkv, nblk * bs, D // 32), generator=g, device=dev,
                      dtype=torch.int32)
    q = torch.randint(-2**31, 2**31 - 1, (T, N, Hq, D // 32), generator=g, device=dev, dtype=torch.int32)
    tables = torch.randperm(nblk, generator=torch.Generator().manual_seed(4))[:N * 8].view(N, 8)
    tables = tables.to(torch.int32).to(dev)
    lens = torch.tensor([1, 17, 64, 100, 128], dtype=torch.int32, device=dev)
    got = paged_spike_attn_decode(q, k, v, tables, lens, D, bs, Hq, Hkv)
    want = paged_spike_attn_decode_cpu(q.cpu(), k.cpu(), v.cpu(), tables.cpu(), lens.cpu(), D, bs, Hq, Hkv)
    torch.cuda.synchronize(dev)
    err = float((got.cpu() - want).abs().max())
    ok = err <= 1e-3
    return Check("decode attention", "ok" if ok else "fail",
                 f"max-abs {err:.2e} against paged_spike_attn_decode_cpu (limit 1e-3)", {"max_abs": err})


def check_kernels(device: torch.device | str | None = None) -> list[Check]:
    """The library check, then (on a GPU) the packing, LIF and decode
    attention checks, in order; a check that raises reports ``fail``."""
    checks = [_library()]
    has_gpu = torch.cuda.is_available()
    if not has_gpu or checks[0].status != "ok":
        why = "no GPU visible" if not has_gpu else "the library did not load"
        checks += [Check(n, "skip", why) for n in ("packing round trip", "lif kernel", "decode attention")]
        return checks
    dev = torch.device(device) if device is not None else torch.device("cuda:0")
    for fn, name in ((_packing, "packing round trip"), (_lif, "lif kernel"), (_attention, "decode attention")):
        try:
            checks.append(fn(dev))
        except Exception as exc:
            checks.append(Check(name, "fail", f"{type(exc).__name__}: {exc}"))
    return checks


def main() -> int:
    checks = check_kernels()
    width = max(len(c.name) for c in checks)
    for c in checks:
        print(f"{c.name:<{width}}  {c.status:<4}  {c.detail}")
    return 1 if any(c.status == "fail" for c in checks) else 0


if __name__ == "__main__":
    sys.exit(main())
