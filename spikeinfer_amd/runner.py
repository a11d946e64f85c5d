"""Batched generation: eager prefill, then decode steps replayed from one
captured hipGraph (counterpart of spikeinfer/engine/model_runner.py:66-287).

The reference replays a captured forward and goes back to the host every step
to sample and to rebuild positions, slots and sequence lengths.  Here the graph
holds the whole step -- forward, lm_head, sampling, and the advance of every
row to its next position -- so consecutive replays need no host work at all.
Static buffers follow the reference's capture conventions
(model_runner.py:189-287): rows past the live batch point at the cache's pad
block with ``seq_len = 1`` and never advance.  As there, one graph is captured
per batch bucket (config.py:117-126: 1, 2, 4, ..., 64) and a batch runs in the
smallest bucket that holds it; every bucket's graph works on a row prefix of
the same static buffers, and all of them share one graph memory pool.
"""
from __future__ import annotations

import math

import torch

from .attention import AttentionMetadata
from .kernels.decoder_ops import decode_advance
from .model import SpikingDecoder
from .sampler import BatchSampler, SamplingParams, sample_tokens
from .spike_cache import PagedSpikeCache, slot_mapping


DEFAULT_BUCKETS = (1, 2, 4, 8, 16, 32, 64)


class DecodeRunner:
    def __init__(self, model: SpikingDecoder, cache: PagedSpikeCache, batch_size: int,
                 max_model_len: int, max_new_tokens: int = 2048,
                 buckets: tuple[int, ...] = DEFAULT_BUCKETS, batched_prefill: bool = False) -> None:
        # batched_prefill: one prefill forward over all prompts (fewer, larger
        # GEMMs) instead of one per prompt.  The library GEMMs of a prefill may
        # then round a row differently with the batch around it, so tokens can
        # depend on the batch; per-prompt prefill keeps them batch-invariant.
        self.batched_prefill = batched_prefill
        self.model = model
        self.cache = cache
        self.B = batch_size
        self.bs = cache.block_size
        self.max_blocks = math.ceil(max_model_len / self.bs)
        dev = self.device = model.device
        c = model.config
        self.input_ids = torch.zeros(batch_size, dtype=torch.int64, device=dev)
        self.positions = torch.zeros(batch_size, dtype=torch.int64, device=dev)
        self.slot_mapping = torch.full((batch_size,), cache.pad_slot, dtype=torch.int64, device=dev)
        self.block_tables = torch.full((batch_size, self.max_blocks), cache.pad_block,
                                       dtype=torch.int32, device=dev)
        self.seq_lens = torch.ones(batch_size, dtype=torch.int32, device=dev)
        self.meta = self._meta(batch_size)
        # Buckets up to the batch size; the batch size itself is always one, so
        # every live count up to it has a graph.
        self.buckets = tuple(sorted({b for b in buckets if 0 < b < batch_size} | {batch_size}))
        self._bufs: dict[int, dict[str, torch.Tensor]] = {}
        self.logits = torch.empty((batch_size, c.vocab_size), dtype=model.dtype, device=dev)
        self.sampler = BatchSampler(batch_size, dev)
        self.history = torch.zeros((batch_size, max_new_tokens), dtype=torch.int64, device=dev)
        self.step_count = torch.zeros(1, dtype=torch.int32, device=dev)
        self.live = torch.zeros(1, dtype=torch.int32, device=dev)  # rows that advance
        self.n_live = 0
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.graph_stages: dict[int, int] = {}  # sampler stages each graph was captured with
        self._free_blocks = list(range(cache.num_allocatable_blocks))

    def _meta(self, b: int) -> AttentionMetadata:
        return AttentionMetadata(slot_mapping=self.slot_mapping[:b], block_size=self.bs,
                                 num_decode_tokens=b, block_tables=self.block_tables[:b],
                                 seq_lens=self.seq_lens[:b])

    def bucket_for(self, n: int) -> int:
        """Smallest bucket holding ``n`` rows (model_runner.py:180-184)."""
        for b in self.buckets:
            if b >= n:
                return b
        raise ValueError(f"batch of {n} exceeds the runner's {self.B} rows")

    # -- one decode step (the captured body) ------------------------------------
    def _step(self, b: int | None = None) -> None:
        """One decode step over rows ``[0, b)`` (default: the whole batch)."""
        b = self.B if b is None else b
        m, s = self.model, self.sampler
        if b not in self._bufs:
            self._bufs[b] = {
                "q_packed": torch.empty((m.T, b, m.Hq, m.W), dtype=torch.int32, device=self.device),
                "attn": torch.empty((m.T, b, m.Hq, m.D), dtype=m.dtype, device=self.device),
            }
        meta = self.meta if b == self.B else self._meta(b)
        hidden = m.forward_paged(self.input_ids[:b], self.positions[:b], self.cache.layers, meta,
                                 self._bufs[b])
        logits = self.logits[:b]
        m.compute_logits(hidden, out=logits)
        # s.uniforms holds this step's draws: written by the previous step's
        # decode_advance (no torch RNG in the captured step)
        sample_tokens(logits, s.temperature[:b], s.top_k[:b], s.top_p[:b], s.min_p[:b],
                      s.repetition_penalty[:b], s.presence_penalty[:b], s.frequency_penalty[:b],
                      self.history, self.step_count, s.uniforms[:b], s.tokens[:b], workspace=s.workspace,
                      stages=s.stages)
        decode_advance(s.tokens, self.input_ids, self.positions, self.seq_lens, self.slot_mapping,
                       self.block_tables, self.bs, b, self.live, self.history, self.step_count,
                       s.rng_seeds, s.uniforms)

    # -- prefill -------------------------------------------------------------
    @torch.no_grad()
    def start(self, prompts: list[list[int]], params: list[SamplingParams],
              shuffle_blocks: int | None = None) -> None:
        """Allocates blocks, runs the prompts through an eager prefill (one
        forward per prompt, or one for all with ``batched_prefill``), samples
        each row's first token and leaves the static buffers pointing at the
        first decode step.  ``shuffle_blocks`` seeds a random physical block
        order (the reference's block manager hands out whatever is free)."""
        n = len(prompts)
        if n > self.B or len(params) != n:
            raise ValueError(f"{n} prompts for a batch of {self.B} ({len(params)} params)")
        free = list(self._free_blocks)
        if shuffle_blocks is not None:
            g = torch.Generator().manual_seed(shuffle_blocks)
            free = [free[i] for i in torch.randperm(len(free), generator=g).tolist()]
        tables, ids, pos, slots, starts = [], [], [], [], []
        for p in prompts:
            need = self.max_blocks
            if need > len(free):
                raise ValueError("cache too small for the batch at max_model_len")
            tab, free = free[:need], free[need:]
            tables.append(tab)
            starts.append(len(ids))
            ids += p
            pos += range(len(p))
            slots += slot_mapping(tab, 0, len(p), self.bs)
        dev = self.device

        def prefill(group):  # prompt indices -> their last tokens' hidden rows
            off, ss, ii, pp, sl = 0, [], [], [], []
            for k in group:
                ss.append(off)
                ii += prompts[k]
                pp += range(len(prompts[k]))
                sl += slots[starts[k]:starts[k] + len(prompts[k])]
                off += len(prompts[k])
            meta = AttentionMetadata(
                slot_mapping=torch.tensor(sl, dtype=torch.int64, device=dev), block_size=self.bs,
                num_decode_tokens=0, prefill_query_starts=ss,
                prefill_query_lens=[len(prompts[k]) for k in group], prefill_context_lens=[0] * len(group),
                prefill_block_tables=[torch.tensor(tables[k], dtype=torch.int32, device=dev) for k in group])
            hidden = self.model.forward_paged(torch.tensor(ii, dtype=torch.int64, device=dev),
                                              torch.tensor(pp, dtype=torch.int64, device=dev),
                                              self.cache.layers, meta)
            last = torch.tensor([s + len(prompts[k]) - 1 for s, k in zip(ss, group)], device=dev)
            return hidden.index_select(0, last)

        if self.batched_prefill:
            rows = prefill(list(range(n)))
        else:
            rows = torch.cat([prefill([k]) for k in range(n)])
        logits = self.model.compute_logits(rows)

        self.live.fill_(n)
        self.n_live = n
        self.sampler.set_params(params)
        self.block_tables.fill_(self.cache.pad_block)
        self.block_tables[:n] = torch.tensor(tables, dtype=torch.int32, device=dev)
        self.positions.zero_()
        self.positions[:n] = torch.tensor([len(p) - 1 for p in prompts], device=dev)
        self.seq_lens.fill_(1)
        self.slot_mapping.fill_(self.cache.pad_slot)
        self.input_ids.zero_()
        self.step_count.zero_()
        self.history.zero_()
        s = self.sampler
        s.draw_uniforms(n)
        sample_tokens(logits, s.temperature[:n], s.top_k[:n], s.top_p[:n], s.min_p[:n],
                      s.repetition_penalty[:n], s.presence_penalty[:n], s.frequency_penalty[:n],
                      self.history, self.step_count, s.uniforms[:n], s.tokens[:n], workspace=s.workspace,
                      stages=s.stages)
        decode_advance(s.tokens, self.input_ids, self.positions, self.seq_lens, self.slot_mapping,
                       self.block_tables, self.bs, self.B, self.live, self.history, self.step_count,
                       s.rng_seeds, s.uniforms)

    # -- capture and replay --------------------------------------------------------
    @torch.no_grad()
    def capture(self, buckets: tuple[int, ...] | None = None) -> list[int]:
        """Captures one decode step per bucket (default: all of them), largest
        first into one shared memory pool.  Warm-up runs on the pad block only
        (the live rows are parked and restored), so capture changes no
        sequence.  A graph keeps the sampler's sliced stages of the requests
        at capture (other requests replay it with the same tokens, perhaps
        slower; :meth:`replay` recaptures).  Returns the buckets captured."""
        todo = sorted(self.buckets if buckets is None else buckets, reverse=True)
        for b in todo:
            if b not in self.buckets:
                raise ValueError(f"{b} is not one of the buckets {self.buckets}")
        parked = (self.input_ids, self.positions, self.seq_lens, self.slot_mapping,
                  self.step_count, self.history, self.live, self.sampler.tokens,
                  self.sampler.uniforms)
        saved = [t.clone() for t in parked]
        self.live.zero_()
        bt = self.block_tables.clone()
        self.block_tables.fill_(self.cache.pad_block)
        self.slot_mapping.fill_(self.cache.pad_slot)
        self.seq_lens.fill_(1)
        self.positions.zero_()
        stream = torch.cuda.Stream(self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            for b in todo:
                for _ in range(2):
                    self._step(b)
        torch.cuda.current_stream(self.device).wait_stream(stream)
        torch.cuda.synchronize(self.device)
        pool = None
        for b in todo:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                self._step(b)
            pool = g.pool()
            self.graphs[b] = g
            self.graph_stages[b] = self.sampler.stages
        self.block_tables.copy_(bt)
        for t, v in zip(parked, saved):
            t.copy_(v)
        return todo

    @property
    def graph(self) -> torch.cuda.CUDAGraph | None:
        """The graph the live batch replays (None before its bucket is captured)."""
        return self.graphs.get(self.bucket_for(max(self.n_live, 1)))

    def replay(self, steps: int = 1) -> None:
        """Replays the live batch's graph `steps` times.  The graph is
        recaptured first when the live requests need other sampler stages than
        the ones it was captured with (the tokens would not change, but the
        captured stages would run the wrong kernels for these requests)."""
        b = self.bucket_for(max(self.n_live, 1))
        if b in self.graphs and self.graph_stages.get(b) != self.sampler.stages:
            self.capture((b,))
        g = self.graph
        if g is None:
            raise RuntimeError(f"no graph captured for a batch of {self.n_live}")
        for _ in range(steps):
            g.replay()

    @torch.no_grad()
    def generate(self, prompts: list[list[int]], params: list[SamplingParams],
                 max_new_tokens: int, shuffle_blocks: int | None = None) -> torch.Tensor:
        """``[n, max_new_tokens]`` generated token ids (first from prefill).

        Raises ValueError when ``max_new_tokens`` exceeds the history the
        runner was built with (its ``max_new_tokens`` argument).
        """
        if max_new_tokens > self.history.shape[1]:
            raise ValueError(
                f"max_new_tokens={max_new_tokens} exceeds the runner's history of "
                f"{self.history.shape[1]} tokens (construct it with a larger max_new_tokens)")
        self.start(prompts, params, shuffle_blocks)
        b = self.bucket_for(len(prompts))
        if self.graph is None:
            self.capture((b,))
        self.replay(max_new_tokens - 1)
        return self.history[: len(prompts), :max_new_tokens].clone()
