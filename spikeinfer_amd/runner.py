"""Batched generation: eager prefill, then decode steps replayed from one
captured hipGraph (counterpart of spikeinfer/engine/model_runner.py:66-287).

The reference replays a captured forward and goes back to the host every step
to sample and to rebuild positions, slots and sequence lengths.  Here the graph
holds the whole step -- forward, lm_head, sampling, and the advance of every
row to its next position -- so consecutive replays need no host work at all.
Static buffers follow the reference's capture conventions
(model_runner.py:189-287): rows past the live batch point at the cache's pad
block with ``seq_len = 1`` and never advance.
"""
from __future__ import annotations

import math

import torch

from .attention import AttentionMetadata
from .kernels.decoder_ops import decode_advance
from .model import SpikingDecoder
from .sampler import BatchSampler, SamplingParams, sample_tokens
from .spike_cache import PagedSpikeCache, slot_mapping


class DecodeRunner:
    def __init__(self, model: SpikingDecoder, cache: PagedSpikeCache, batch_size: int,
                 max_model_len: int, max_new_tokens: int = 2048) -> None:
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
        self.meta = AttentionMetadata(slot_mapping=self.slot_mapping, block_size=self.bs,
                                      num_decode_tokens=batch_size, block_tables=self.block_tables,
                                      seq_lens=self.seq_lens)
        self.bufs = {
            "q_packed": torch.empty((model.T, batch_size, model.Hq, model.W), dtype=torch.int32, device=dev),
            "attn": torch.empty((model.T, batch_size, model.Hq, model.D), dtype=model.dtype, device=dev),
        }
        self.logits = torch.empty((batch_size, c.vocab_size), dtype=model.dtype, device=dev)
        self.sampler = BatchSampler(batch_size, dev)
        self.history = torch.zeros((batch_size, max_new_tokens), dtype=torch.int64, device=dev)
        self.step_count = torch.zeros(1, dtype=torch.int32, device=dev)
        self.live = torch.zeros(1, dtype=torch.int32, device=dev)  # rows that advance
        self.graph: torch.cuda.CUDAGraph | None = None
        self._free_blocks = list(range(cache.num_allocatable_blocks))

    # -- one decode step (the captured body) ------------------------------------
    def _step(self) -> None:
        m, s = self.model, self.sampler
        hidden = m.forward_paged(self.input_ids, self.positions, self.cache.layers, self.meta, self.bufs)
        m.compute_logits(hidden, out=self.logits)
        s.uniforms.uniform_()
        sample_tokens(self.logits, s.temperature, s.top_k, s.top_p, s.min_p, s.repetition_penalty,
                      s.presence_penalty, s.frequency_penalty, self.history, self.step_count,
                      s.uniforms, s.tokens)
        decode_advance(s.tokens, self.input_ids, self.positions, self.seq_lens, self.slot_mapping,
                       self.block_tables, self.bs, self.B, self.live, self.history, self.step_count)

    # -- prefill -------------------------------------------------------------
    @torch.no_grad()
    def start(self, prompts: list[list[int]], params: list[SamplingParams],
              shuffle_blocks: int | None = None) -> None:
        """Allocates blocks, runs the prompts through one eager prefill, samples
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
        meta = AttentionMetadata(
            slot_mapping=torch.tensor(slots, dtype=torch.int64, device=dev), block_size=self.bs,
            num_decode_tokens=0, prefill_query_starts=starts,
            prefill_query_lens=[len(p) for p in prompts], prefill_context_lens=[0] * n,
            prefill_block_tables=[torch.tensor(t, dtype=torch.int32, device=dev) for t in tables])
        hidden = self.model.forward_paged(torch.tensor(ids, dtype=torch.int64, device=dev),
                                          torch.tensor(pos, dtype=torch.int64, device=dev),
                                          self.cache.layers, meta)
        last = torch.tensor([s + len(p) - 1 for s, p in zip(starts, prompts)], device=dev)
        logits = self.model.compute_logits(hidden, last)

        self.live.fill_(n)
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
                      self.history, self.step_count, s.uniforms[:n], s.tokens[:n])
        decode_advance(s.tokens, self.input_ids, self.positions, self.seq_lens, self.slot_mapping,
                       self.block_tables, self.bs, self.B, self.live, self.history, self.step_count)

    # -- capture and replay --------------------------------------------------------
    @torch.no_grad()
    def capture(self) -> None:
        """Captures one decode step.  Warm-up runs on the pad block only (the
        live rows are parked and restored), so capture changes no sequence."""
        parked = (self.input_ids, self.positions, self.seq_lens, self.slot_mapping,
                  self.step_count, self.history, self.live, self.sampler.tokens)
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
            for _ in range(2):
                self._step()
        torch.cuda.current_stream(self.device).wait_stream(stream)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        self.block_tables.copy_(bt)
        for t, v in zip(parked, saved):
            t.copy_(v)

    def replay(self, steps: int = 1) -> None:
        for _ in range(steps):
            self.graph.replay()

    @torch.no_grad()
    def generate(self, prompts: list[list[int]], params: list[SamplingParams],
                 max_new_tokens: int, shuffle_blocks: int | None = None) -> torch.Tensor:
        """``[n, max_new_tokens]`` generated token ids (first from prefill)."""
        self.start(prompts, params, shuffle_blocks)
        if self.graph is None:
            self.capture()
        self.replay(max_new_tokens - 1)
        return self.history[: len(prompts), :max_new_tokens].clone()
