"""The HIP sampler against the sampler oracle (oracle.sample_row, a numpy
restatement of spikeinfer/engine/sampler.py:48-177) on identical logits and
uniforms.  The kernel's token must be in the oracle's kept set and its
interval of the oracle's CDF (kept tokens by value descending, index
ascending) must contain u (widened by 1e-6, the float32 weights' rounding);
where u is farther than that from every boundary this is the same token as
the oracle's.  Rows whose filter cut lies within
rounding of its boundary (oracle margin < 1e-6) only need a kept token, and
must stay rare."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from spikeinfer_amd.sampler import BatchSampler, SamplingParams, sample_tokens, sample_workspace_bytes

pytestmark = pytest.mark.gpu


def _run(gpu, logits, params, histories, uniforms, dtype=torch.float32, sliced=False):
    n, V = logits.shape
    lg = torch.from_numpy(logits).to(gpu, dtype)
    f = lambda k, dflt: torch.tensor([p.get(k, dflt) for p in params], dtype=torch.float32, device=gpu)
    cap = max(1, max(len(h) for h in histories))
    hist = torch.zeros((n, cap), dtype=torch.int64, device=gpu)
    for i, h in enumerate(histories):
        if h:
            hist[i, :len(h)] = torch.tensor(h)
    hlen = torch.tensor([len(h) for h in histories], dtype=torch.int32, device=gpu)
    out = sample_tokens(
        lg, f("temperature", 1.0),
        torch.tensor([p.get("top_k", -1) for p in params], dtype=torch.int32, device=gpu),
        f("top_p", 1.0), f("min_p", 0.0), f("rep", 1.0), f("presence", 0.0), f("frequency", 0.0),
        hist, hlen, torch.tensor(uniforms, dtype=torch.float32, device=gpu),
        workspace=torch.empty(sample_workspace_bytes(n), dtype=torch.uint8, device=gpu) if sliced else None)
    return out.cpu().tolist(), lg.float().cpu().numpy()


CASES = [
    dict(temperature=0.8, top_k=50, top_p=0.9, rep=1.1),  # config 5
    dict(temperature=1.0),
    dict(temperature=0.7, top_k=1),
    dict(temperature=1.3, top_p=0.5),
    dict(temperature=0.9, min_p=0.05),
    dict(temperature=1.0, top_k=200, min_p=0.01, top_p=0.95),
    dict(temperature=0.5, top_k=10, presence=0.5, frequency=0.25, rep=1.3),
    dict(temperature=0.0, rep=1.5),
    dict(temperature=2.0, top_k=100000),
]


@pytest.mark.parametrize("sliced", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_sampler_matches_oracle(gpu, case, dtype, sliced):
    rng = np.random.default_rng(case)
    rows, V = 16, 151936
    logits = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
    params = [CASES[case]] * rows
    histories = [rng.integers(0, V, size=rng.integers(0, 40)).tolist() for _ in range(rows)]
    # Make some history tokens strong so the penalties matter.
    for i, h in enumerate(histories):
        for t in h[:3]:
            logits[i, t] = 12.0 + rng.standard_normal()
    us = rng.random(rows).astype(np.float32).tolist()
    got, used = _run(gpu, logits, params, histories, us, dtype, sliced)
    skipped = 0
    for i in range(rows):
        p = params[i]
        tok, kept, _probs, margin, order = orc.sample_row(
            used[i], temperature=p.get("temperature", 1.0), top_k=p.get("top_k", -1),
            top_p=p.get("top_p", 1.0), min_p=p.get("min_p", 0.0), rep=p.get("rep", 1.0),
            presence=p.get("presence", 0.0), frequency=p.get("frequency", 0.0),
            history=histories[i], u=us[i])
        if margin < 1e-6:
            skipped += 1
            continue
        t = got[i]
        assert kept[t], f"row {i}: token {t} not kept (oracle {tok})"
        cdf = np.cumsum(_probs[order])
        pos = int(np.nonzero(order == t)[0][0])
        lo, hi = cdf[pos] - _probs[t], cdf[pos]
        assert lo - 1e-6 <= us[i] <= hi + 1e-6, f"row {i}: u={us[i]} outside [{lo}, {hi}] of {t}"
        if lo + 1e-6 < us[i] < hi - 1e-6:
            assert t == tok
    assert skipped <= 2


SLICED_CASES = [
    (151936, 3.0, dict(temperature=0.8, top_k=50, top_p=0.9, rep=1.1)),
    (151936, 3.0, dict(temperature=1.0, top_k=256, min_p=0.02, presence=0.4, frequency=0.3)),
    (151936, 3.0, dict(temperature=1.0, top_k=257)),             # above the sliced range
    (151936, 0.0, dict(temperature=1.0, top_k=50)),              # every logit equal: slices overflow
    (151936, 0.02, dict(temperature=0.7, top_k=8, top_p=0.5)),   # bf16: heavy ties
    (1000, 3.0, dict(temperature=1.0, top_k=50)),                # slices past the vocabulary are empty
    (100, 3.0, dict(temperature=1.0, top_k=60, rep=2.0)),        # one partial slice, k near the vocabulary
    (262144, 3.0, dict(temperature=1.2, top_k=1)),               # the largest vocabulary
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", range(len(SLICED_CASES)))
def test_sampler_sliced_candidates_give_the_same_tokens(gpu, case, dtype):
    """With the workspace, rows with a top-k cut take their candidates from
    the sliced stage (or fall back to the row sweeps when a slice cannot
    certify its set): every token equals the one-workgroup path's."""
    V, scale, p = SLICED_CASES[case]
    print(f"sliced sampler case {case} V={V} dtype={dtype}", flush=True)
    rng = np.random.default_rng(100 + case)
    rows = 24
    logits = (rng.standard_normal((rows, V)) * scale).astype(np.float32)
    histories = [rng.integers(0, V, size=rng.integers(0, 60)).tolist() for _ in range(rows)]
    for i, h in enumerate(histories):
        for t in h[:3]:
            logits[i, t] = 10.0 + rng.standard_normal()
    us = rng.random(rows).astype(np.float32).tolist()
    plain, _ = _run(gpu, logits, [p] * rows, histories, us, dtype)
    sliced, _ = _run(gpu, logits, [p] * rows, histories, us, dtype, sliced=True)
    assert sliced == plain


# Rows with no top-k cut (the open stage).  "peaked" logits are N(0, 6^2) (a
# trained model's kind: the top few hundred tokens hold most of the mass, so
# the slices decide most rows); flat N(0, 2^2) ones leave the cut past the
# slices' lists, and the rows fall back to the one-workgroup path.
OPEN_CASES = [
    (151936, 6.0, dict(temperature=1.0)),                         # no cut at all: not taken by the stage
    (151936, 6.0, dict(temperature=1.0, min_p=0.01)),             # min_p only: the draw over the alive mass
    (151936, 6.0, dict(temperature=0.8, top_p=0.9, rep=1.1)),
    (151936, 6.0, dict(temperature=1.0, min_p=0.05, top_p=0.95, presence=0.4, frequency=0.3)),
    (151936, 6.0, dict(temperature=1.3, top_k=151936, top_p=0.7)),  # top_k >= vocab: no cut
    (151936, 2.0, dict(temperature=1.0, min_p=0.001)),            # flat: falls back
    (151936, 2.0, dict(temperature=1.0, top_p=0.9)),
    (151936, 0.0, dict(temperature=1.0, top_p=0.5)),              # every logit equal
    (151936, 0.05, dict(temperature=0.7, top_p=0.5)),             # bf16: heavy ties
    (1000, 3.0, dict(temperature=1.0, top_p=0.8)),                # four slices, the last one short
    (60, 3.0, dict(temperature=1.0, top_p=0.999, rep=2.0)),       # one slice, listed whole
    (100, 3.0, dict(temperature=1.0, min_p=0.2, rep=2.0)),        # one partial slice
    (262144, 8.0, dict(temperature=1.2, top_p=0.99)),             # the largest vocabulary
    (151936, 30.0, dict(temperature=0.3, top_p=0.99)),            # nearly one-hot
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", range(len(OPEN_CASES)))
def test_sampler_open_rows_give_the_same_tokens(gpu, case, dtype):
    """With the workspace, rows with no top-k cut are decided from the slices'
    lists and exact mass partials when their top-p cut and draw fall inside
    the certified prefix, and by the one-workgroup path otherwise: every token
    equals the one-workgroup path's."""
    V, scale, p = OPEN_CASES[case]
    print(f"open-row sampler case {case} V={V} dtype={dtype}", flush=True)
    rng = np.random.default_rng(200 + case)
    rows = 24
    logits = (rng.standard_normal((rows, V)) * scale).astype(np.float32)
    histories = [rng.integers(0, V, size=rng.integers(0, 60)).tolist() for _ in range(rows)]
    for i, h in enumerate(histories):
        for t in h[:3]:
            logits[i, t] = 4 * scale + rng.standard_normal()
    us = rng.random(rows).astype(np.float32).tolist()
    us[0], us[1] = 0.0, float(np.nextafter(np.float32(1), np.float32(0)))  # the ends of the draw
    plain, _ = _run(gpu, logits, [p] * rows, histories, us, dtype)
    sliced, _ = _run(gpu, logits, [p] * rows, histories, us, dtype, sliced=True)
    assert sliced == plain


def test_sampler_mixed_batch_and_stage_bits(gpu):
    """One batch of open, top-k, greedy and large-k rows: every stage set gives
    the one-workgroup path's tokens, including a workspace last filled by a
    call with other stages (the row kernel reads only the lists this call's
    stages wrote)."""
    from spikeinfer_amd.sampler import STAGE_OPEN, STAGE_TOPK, stages_for

    rng = np.random.default_rng(77)
    rows, V = 32, 151936
    kinds = [dict(temperature=1.0), dict(temperature=0.8, top_k=40, top_p=0.9),
             dict(temperature=0.0), dict(temperature=1.0, top_k=1000), dict(temperature=0.9, top_p=0.8),
             dict(temperature=1.1, top_k=V, top_p=0.95)]
    params = [kinds[i % len(kinds)] for i in range(rows)]
    t = torch.tensor([q["temperature"] for q in params], dtype=torch.float32, device=gpu)
    k = torch.tensor([q.get("top_k", -1) for q in params], dtype=torch.int32, device=gpu)
    tp = torch.tensor([q.get("top_p", 1.0) for q in params], dtype=torch.float32, device=gpu)
    ws = torch.empty(sample_workspace_bytes(rows), dtype=torch.uint8, device=gpu)
    for trial in range(2):
        lg = torch.from_numpy((rng.standard_normal((rows, V)) * 6).astype(np.float32)).to(gpu, torch.bfloat16)
        u = torch.from_numpy(rng.random(rows).astype(np.float32)).to(gpu)
        plain = sample_tokens(lg, t, k, tp, uniforms=u)
        for st in (STAGE_TOPK | STAGE_OPEN, STAGE_TOPK, STAGE_OPEN, 0):
            got = sample_tokens(lg, t, k, tp, uniforms=u, workspace=ws, stages=st)
            assert torch.equal(plain, got), (trial, st)
    sp = [SamplingParams(temperature=q["temperature"], top_k=q.get("top_k", -1), top_p=q.get("top_p", 1.0))
          for q in kinds]
    assert stages_for(sp) == STAGE_TOPK | STAGE_OPEN
    assert stages_for(sp[1:2]) == STAGE_TOPK and stages_for(sp[2:3]) == 0
    assert stages_for(sp[3:4]) == 0 and stages_for(sp[4:5]) == STAGE_OPEN


def test_sampler_workspace_with_unaligned_rows_takes_the_row_path(gpu):
    """Rows whose stride is not a whole number of 16-byte vectors cannot be
    sliced: with a workspace they take the one-workgroup path, same tokens."""
    g = torch.Generator(device=gpu).manual_seed(3)
    wide = torch.randn((12, 1001), generator=g, device=gpu) * 2
    lg = wide[:, :1000]  # row stride 1001 floats
    rows = lg.shape[0]
    t = torch.full((rows,), 0.9, device=gpu)
    k = torch.full((rows,), 20, dtype=torch.int32, device=gpu)
    u = torch.rand(rows, generator=g, device=gpu)
    plain = sample_tokens(lg, t, k, uniforms=u)
    ws = torch.empty(sample_workspace_bytes(rows), dtype=torch.uint8, device=gpu)
    sliced = sample_tokens(lg, t, k, uniforms=u, workspace=ws)
    assert torch.equal(plain, sliced)


def test_sampler_slices_never_read_past_the_row(gpu):
    """A last slice with fewer elements than one 16-byte vector (bf16 V = 515:
    slices of 256, 256 and 3; fp32 V = 258: 256 and 2), aligned rows (so the
    sliced path runs) and a last row that ends its allocation: the sliced and
    one-workgroup paths agree."""
    for V, stride, dt in ((515, 520, torch.bfloat16), (258, 260, torch.float32)):
        g = torch.Generator(device=gpu).manual_seed(V)
        rows = 6
        flat = (torch.randn((rows - 1) * stride + V, generator=g, device=gpu) * 2).to(dt)
        lg = flat.as_strided((rows, V), (stride, 1))
        t = torch.full((rows,), 1.0, device=gpu)
        k = torch.full((rows,), 5, dtype=torch.int32, device=gpu)
        u = torch.rand(rows, generator=g, device=gpu)
        plain = sample_tokens(lg, t, k, uniforms=u)
        ws = torch.empty(sample_workspace_bytes(rows), dtype=torch.uint8, device=gpu)
        sliced = sample_tokens(lg, t, k, uniforms=u, workspace=ws)
        assert torch.equal(plain, sliced), (V, dt)


def test_sampler_ties_and_tiny_vocab(gpu):
    """bf16-style ties at the top-k cut are kept in index order."""
    logits = np.array([[1.0, 3.0, 3.0, 3.0, 0.0, 3.0]] * 4, np.float32)
    params = [dict(temperature=1.0, top_k=2)] * 4
    us = [0.0, 0.49, 0.51, 0.999]
    for sliced in (False, True):
        got, _ = _run(gpu, logits, params, [[]] * 4, us, sliced=sliced)
        assert got == [1, 1, 2, 2]


def test_sampler_uniform_sweep_follows_closed_form(gpu):
    """logits ln(1..4): drawn largest first, boundaries at 0.4, 0.7, 0.9."""
    lg = np.log(np.arange(1, 5, dtype=np.float64)).astype(np.float32)
    us = [0.05, 0.39, 0.41, 0.69, 0.71, 0.89, 0.91, 0.99]
    got, _ = _run(gpu, np.stack([lg] * len(us)), [dict()] * len(us), [[]] * len(us), us)
    assert got == [3, 3, 2, 2, 1, 1, 0, 0]


def test_sampler_history_len_shared_count(gpu):
    """history_len with one entry applies the same count to every row."""
    V = 64
    lg = torch.zeros((3, V), device=gpu)
    lg[:, 7] = 5.0
    lg[:, 9] = 4.0
    hist = torch.tensor([[7, 1], [2, 3], [7, 7]], device=gpu)
    t = torch.zeros(3, device=gpu)  # greedy
    rep = torch.full((3,), 2.0, device=gpu)
    one = torch.tensor([1], dtype=torch.int32, device=gpu)
    out = sample_tokens(lg, t, repetition_penalty=rep, history=hist, history_len=one)
    assert out.tolist() == [9, 7, 9]


def test_batch_sampler_records_and_penalises(gpu):
    V = 32
    bsz = BatchSampler(2, gpu, history_cap=8)
    bsz.set_params([SamplingParams(temperature=0.0, repetition_penalty=10.0),
                    SamplingParams(temperature=0.0)])
    lg = torch.zeros((2, V), device=gpu)
    lg[:, 3] = 2.0
    lg[:, 4] = 1.0
    first = bsz.sample(lg).tolist()
    second = bsz.sample(lg).tolist()
    assert first == [3, 3] and second == [4, 3]
    assert bsz.history_len.tolist() == [2, 2]


def test_sampler_rejects_bad_arguments(gpu):
    lg = torch.zeros((2, 10), device=gpu)
    with pytest.raises(ValueError):
        sample_tokens(lg, torch.ones(2, dtype=torch.float64, device=gpu))
    with pytest.raises(ValueError):
        sample_tokens(lg.t(), torch.ones(10, device=gpu))
    with pytest.raises(ValueError):
        SamplingParams(top_k=0)
