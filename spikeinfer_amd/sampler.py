"""Batched on-device sampling (counterpart of spikeinfer/engine/sampler.py).

One HIP launch per step: penalties, temperature, min_p, top_k, top_p and the
draw for every row at once (see ``spk_sample`` in include/spikeinfer_amd.h).
Parameters live in device arrays, so a captured decode step can sample inside
the graph and the parameters can change between replays.

Differences from the reference that a caller can observe:
  * equal logits are ordered by index (the reference leaves that to
    ``torch.topk``), so which of two tied tokens a top-k/top-p cut keeps is
    fixed;
  * the draw is the inverse CDF of the kept weights, tokens taken by value
    descending (index ascending on ties), at a uniform ``u`` that the caller
    supplies (``torch.rand`` by default, a per-request ``torch.Generator`` for
    seeded requests), where the reference calls ``torch.multinomial``: the
    same distribution, a different stream.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _lib

_GREEDY_TEMP = 1e-5


def seed_as_int64(seed: int) -> int:
    """A request seed as the int64 the device generator state holds: reduced
    modulo 2**64 (as ``torch.Generator.manual_seed`` accepts any such value)
    and stored as its two's-complement signed value."""
    s = int(seed) & (2 ** 64 - 1)
    return s - 2 ** 64 if s >= 2 ** 63 else s


@dataclass
class SamplingParams:
    """The sampling fields of spikeinfer/sampling_params.py:15-70, same
    defaults and the same validation errors."""

    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = -1
    min_p: float = 0.0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    seed: int | None = None
    logit_bias: dict[int, float] | None = None
    min_tokens: int = 0
    stop_token_ids: list[int] = field(default_factory=list)

    def __post_init__(self) -> None:
        if self.temperature < 0:
            raise ValueError("temperature must be >= 0")
        if not 0 < self.top_p <= 1:
            raise ValueError("top_p must be in (0, 1]")
        if self.top_k < -1 or self.top_k == 0:
            raise ValueError("top_k must be -1 (disabled) or >= 1")
        if not 0 <= self.min_p <= 1:
            raise ValueError("min_p must be in [0, 1]")
        if self.repetition_penalty <= 0:
            raise ValueError("repetition_penalty must be > 0")

    @property
    def is_greedy(self) -> bool:
        return self.temperature < _GREEDY_TEMP


# Sliced stages of sample_tokens (spk_sample_ws's SPK_SAMPLE_STAGE_* bits).
STAGE_TOPK = 1
STAGE_OPEN = 2
_SLICED_MAX_K = 256  # largest top_k of the top-k stage


def stages_for(params: list["SamplingParams"]) -> int:
    """The sliced stages a batch of these requests can use: the top-k stage
    for sampled rows with 0 < top_k <= 256, the open stage for sampled rows
    with any other top_k (no cut, or one at least the vocabulary) and a top-p
    or min-p cut."""
    st = 0
    for p in params:
        if p.is_greedy:
            continue
        if 0 < p.top_k <= _SLICED_MAX_K:
            st |= STAGE_TOPK
        elif p.top_p < 1.0 or p.min_p > 0.0:
            st |= STAGE_OPEN
    return st


def sample_tokens(
    logits: torch.Tensor,
    temperature: torch.Tensor,
    top_k: torch.Tensor | None = None,
    top_p: torch.Tensor | None = None,
    min_p: torch.Tensor | None = None,
    repetition_penalty: torch.Tensor | None = None,
    presence_penalty: torch.Tensor | None = None,
    frequency_penalty: torch.Tensor | None = None,
    history: torch.Tensor | None = None,
    history_len: torch.Tensor | None = None,
    uniforms: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    stages: int = STAGE_TOPK | STAGE_OPEN,
) -> torch.Tensor:
    """One token per row of ``logits [rows, vocab]`` (fp32/bf16/fp16, row
    stride free, vocab stride 1).

    Per-row device arrays (``rows`` entries): ``temperature`` float32,
    ``top_k`` int32 (-1 off), ``top_p``/``min_p``/penalties float32 (None =
    off).  ``history`` int64 ``[rows, cap]`` holds each row's generated tokens,
    ``history_len`` int32 ``[rows]`` (or ``[1]``: one count for all rows) how
    many.  ``uniforms`` float32 ``[rows]`` in [0, 1) drive the draw.  Returns
    ``out`` int64 ``[rows]``.  ``workspace`` (uint8, at least
    :func:`sample_workspace_bytes` ``(rows)``) lets rows spread their
    candidate search over several workgroups per row, with the same tokens:
    ``stages`` bit :data:`STAGE_TOPK` for rows with 0 < top_k <= 256, bit
    :data:`STAGE_OPEN` for rows with no top-k cut and a top-p or min-p cut
    (each stage costs its launches whether or not the batch holds such rows;
    :func:`stages_for` picks them for a batch of requests).
    """
    dev = _lib.require_gpu(logits, temperature, top_k, top_p, min_p, repetition_penalty,
                           presence_penalty, frequency_penalty, history, history_len, uniforms, out)
    if logits.ndim != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [rows, vocab] with a contiguous vocab axis")
    rows, vocab = logits.shape
    checks = (("temperature", temperature, torch.float32), ("top_k", top_k, torch.int32),
              ("top_p", top_p, torch.float32), ("min_p", min_p, torch.float32),
              ("repetition_penalty", repetition_penalty, torch.float32),
              ("presence_penalty", presence_penalty, torch.float32),
              ("frequency_penalty", frequency_penalty, torch.float32),
              ("uniforms", uniforms, torch.float32))
    for name, t, dt in checks:
        if t is not None and (t.dtype != dt or t.numel() < rows or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous {dt} tensor of {rows} entries")
    hist_stride = len_stride = 0
    if history is not None:
        if history_len is None or history.dtype != torch.int64 or history.ndim != 2 \
                or not history.is_contiguous() or history.shape[0] < rows:
            raise ValueError("history must be contiguous int64 [rows, cap] with history_len")
        if history_len.dtype != torch.int32:
            raise ValueError("history_len must be int32")
        hist_stride = history.stride(0)
        len_stride = 0 if history_len.numel() == 1 else 1
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=dev)
    ws_bytes = 0
    if workspace is not None:
        ws_bytes = workspace.numel() * workspace.element_size()
        if not workspace.is_contiguous() or workspace.device != dev:
            raise ValueError("workspace must be a contiguous tensor on the logits' device")
    _lib.check(
        _lib.load().spk_sample_ws(
            logits.data_ptr(), _lib.dtype_code(logits.dtype), logits.stride(0), rows, vocab,
            temperature.data_ptr(), _lib.ptr(top_k), _lib.ptr(top_p), _lib.ptr(min_p),
            _lib.ptr(repetition_penalty), _lib.ptr(presence_penalty), _lib.ptr(frequency_penalty),
            _lib.ptr(history), hist_stride, _lib.ptr(history_len), len_stride, _lib.ptr(uniforms),
            out.data_ptr(), _lib.ptr(workspace), ws_bytes, int(stages), _lib.stream_of(dev),
        ),
        "sample",
    )
    return out


def sample_workspace_bytes(rows: int) -> int:
    """Bytes of the :func:`sample_tokens` workspace for ``rows`` rows."""
    return int(_lib.load().spk_sample_workspace_bytes(rows))


class BatchSampler:
    """Device-resident sampling state for a batch of up to ``max_rows`` rows.

    ``set_params`` fills the per-row arrays from :class:`SamplingParams`; the
    arrays keep their addresses, so a graph that captured :meth:`sample` sees
    new values on replay.  Generated tokens are tracked in ``history`` /
    ``history_len`` for the penalties (spikeinfer/engine/sequence.py:113 counts
    output tokens only).
    """

    def __init__(self, max_rows: int, device: torch.device, history_cap: int = 2048,
                 eos_token_id: int | None = None) -> None:
        self.max_rows = max_rows
        self.device = torch.device(device)
        self.eos_token_id = eos_token_id
        f32 = dict(dtype=torch.float32, device=self.device)
        self.temperature = torch.ones(max_rows, **f32)
        self.top_k = torch.full((max_rows,), -1, dtype=torch.int32, device=self.device)
        self.top_p = torch.ones(max_rows, **f32)
        self.min_p = torch.zeros(max_rows, **f32)
        self.repetition_penalty = torch.ones(max_rows, **f32)
        self.presence_penalty = torch.zeros(max_rows, **f32)
        self.frequency_penalty = torch.zeros(max_rows, **f32)
        self.history = torch.zeros((max_rows, history_cap), dtype=torch.int64, device=self.device)
        self.history_len = torch.zeros(max_rows, dtype=torch.int32, device=self.device)
        self.uniforms = torch.zeros(max_rows, **f32)
        # per-row seeds of the device-side draws of captured steps (decode_advance)
        self.rng_seeds = torch.zeros(max_rows, dtype=torch.int64, device=self.device)
        self.tokens = torch.zeros(max_rows, dtype=torch.int64, device=self.device)
        # candidates of the sliced top-k stage (sample_tokens' workspace)
        self.workspace = torch.empty(sample_workspace_bytes(max_rows), dtype=torch.uint8, device=self.device)
        self.stages = 0  # sliced stages the current requests use (stages_for)
        self.params: list[SamplingParams] = []
        self._generators: dict[int, torch.Generator] = {}

    def set_params(self, params: list[SamplingParams]) -> None:
        if len(params) > self.max_rows:
            raise ValueError(f"{len(params)} rows > max_rows {self.max_rows}")
        n = len(params)
        self.params = list(params)
        self.stages = stages_for(self.params)
        host = lambda vals, dt: torch.tensor(vals, dtype=dt).to(self.device)
        self.temperature[:n] = host([p.temperature for p in params], torch.float32)
        self.top_k[:n] = host([p.top_k for p in params], torch.int32)
        self.top_p[:n] = host([p.top_p for p in params], torch.float32)
        self.min_p[:n] = host([p.min_p for p in params], torch.float32)
        self.repetition_penalty[:n] = host([p.repetition_penalty for p in params], torch.float32)
        self.presence_penalty[:n] = host([p.presence_penalty for p in params], torch.float32)
        self.frequency_penalty[:n] = host([p.frequency_penalty for p in params], torch.float32)
        # seeded rows draw the same sequence whatever else is in the batch; the
        # others take seeds from torch's host generator
        fresh = torch.randint(0, 2 ** 62, (n,), dtype=torch.int64).tolist()
        self.rng_seeds[:n] = host([seed_as_int64(p.seed) if p.seed is not None else fresh[i]
                                   for i, p in enumerate(params)], torch.int64)
        self.history_len.zero_()
        self._generators = {}

    def draw_uniforms(self, n: int) -> None:
        """Fresh uniforms: torch's device RNG, or per-request generators for
        seeded rows (reproducible whatever else is in the batch)."""
        self.uniforms[:n].uniform_()
        for i, p in enumerate(self.params[:n]):
            if p.seed is not None:
                gen = self._generators.get(i)
                if gen is None:
                    gen = torch.Generator(device=self.device)
                    gen.manual_seed(int(p.seed))
                    self._generators[i] = gen
                self.uniforms[i:i + 1].uniform_(generator=gen)

    def _pre_filter(self, logits: torch.Tensor, n: int) -> torch.Tensor:
        """Logit bias and the min_tokens EOS block (sampler.py:87-96, :121-127),
        applied on an fp32 copy only when a row asks for them."""
        need = [i for i, p in enumerate(self.params[:n]) if p.logit_bias or p.min_tokens]
        if not need:
            return logits
        logits = logits.float()
        lens = self.history_len[:n].tolist()  # host sync: only on this rare path
        for i in need:
            p = self.params[i]
            if p.logit_bias:
                idx = torch.tensor(list(p.logit_bias), device=logits.device, dtype=torch.long)
                val = torch.tensor(list(p.logit_bias.values()), device=logits.device)
                logits[i].index_add_(0, idx, val)
            if p.min_tokens and lens[i] < p.min_tokens:
                eos = list(p.stop_token_ids) + ([self.eos_token_id] if self.eos_token_id is not None else [])
                for tid in eos:
                    if 0 <= tid < logits.shape[1]:
                        logits[i, tid] = float("-inf")
        return logits

    def sample(self, logits: torch.Tensor, record: bool = True) -> torch.Tensor:
        """Samples one token per row of ``logits [n, vocab]`` into
        ``self.tokens[:n]`` and (``record``) appends it to the history."""
        n = logits.shape[0]
        logits = self._pre_filter(logits, n)
        sample_tokens(
            logits, self.temperature[:n], self.top_k[:n], self.top_p[:n], self.min_p[:n],
            self.repetition_penalty[:n], self.presence_penalty[:n], self.frequency_penalty[:n],
            self.history[:n], self.history_len[:n], self.uniforms[:n], self.tokens[:n],
            workspace=self.workspace, stages=self.stages,
        )
        if record:
            self.record(n)
        return self.tokens[:n]

    def record(self, n: int) -> None:
        """Appends ``tokens[:n]`` to the history on the device."""
        cap = self.history.shape[1]
        pos = self.history_len[:n].clamp(max=cap - 1).to(torch.int64)
        self.history[:n].scatter_(1, pos[:, None], self.tokens[:n, None])
        self.history_len[:n] += 1
