"""The kernel self-check (the reference's doctor gate, diagnostics.py:289-333):
on a host without a GPU it loads the library and skips the kernel checks; on
an MI355X every check passes, and a broken comparison reports ``fail``."""
from __future__ import annotations

import pytest
import torch

from spikeinfer_amd import diagnostics


def test_diagnostics_without_a_gpu(monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    checks = diagnostics.check_kernels()
    assert [c.name for c in checks] == ["library", "packing round trip", "lif kernel", "decode attention"]
    assert checks[0].status == "ok"
    assert all(c.status == "skip" for c in checks[1:])
    assert diagnostics.main() == 0


@pytest.mark.gpu
def test_diagnostics_on_the_gpu(gpu):
    print("diagnostics: all kernel checks", flush=True)
    checks = diagnostics.check_kernels(gpu)
    assert [c.status for c in checks] == ["ok"] * 4, [(c.name, c.detail) for c in checks]
    assert checks[2].data["exact"] and checks[3].data["max_abs"] <= 1e-3


@pytest.mark.gpu
def test_diagnostics_reports_a_mismatch(gpu, monkeypatch):
    """A LIF yardstick that disagrees is reported, not raised."""
    from spikeinfer_amd import kernels

    real = kernels.lif_multistep_ref

    def off_by_one(x, beta, th, *a, **k):
        s, u = real(x, beta, th, *a, **k)
        s = s.clone()
        s.view(-1)[0] = 1 - s.view(-1)[0]
        return s, u

    monkeypatch.setattr(kernels, "lif_multistep_ref", off_by_one)
    lif = [c for c in diagnostics.check_kernels(gpu) if c.name == "lif kernel"][0]
    assert lif.status == "fail" and "1 spikes differ" in lif.detail
