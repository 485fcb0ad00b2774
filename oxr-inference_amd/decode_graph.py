"""HIP-graph capture and replay of the speculative verify step.

Three entry points:

- :class:`DecodeGraphs` is the one-token decode step (oxr_runtime/decode_graph.py:33-119): host lists
  in, ``(logits, greedy ids)`` out, one graph per batch bucket, padded rows on a scratch page.
- :class:`ExtendGraphs` keeps the reference's interface (oxr_runtime/decode_graph.py:122-205):
  host lists in, greedy ids ``[n, S]`` out, one graph per batch bucket (1, 2, 4, 8, max).
  Padded rows of a bucket write the first S slots of a scratch page and attend only to
  them, as the reference does (decode_graph.py:188-197).
- :class:`VerifyLoop` is the whole step with nothing on the host: drafting and row assembly
  (engine.py:674-710), the 28-layer forward, LM head + argmax, acceptance and length/history
  rollback (engine.py:729-737) -- one graph, replayed back to back.  Histories, lengths and
  block tables stay in device memory; the next replay drafts from the tokens the previous
  one committed.

Graphs are captured on an ordinary stream (default priority).  The reference captures on a
high-priority stream (decode_graph.py:14-17); stream priorities are avoided here.
"""

from __future__ import annotations

import numpy as np
import torch

from . import lm_head, speculative
from .kv_cache import KVCache, pack_page_table
from .language import DecodeBatch, ExtendBatch, LanguageModel, StepBuffers

BUCKETS = (1, 2, 4, 8, 16, 32, 64)  # decode_graph.py:30, up to what the weight-streaming kernels take
EXTEND_BUCKETS = (1, 2, 4, 8)  # decode_graph.py:122


def _warm_up(stream: torch.cuda.Stream, forward, times: int = 2) -> None:
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(times):
            forward()
    torch.cuda.current_stream().wait_stream(stream)


class DecodeGraphs:
    """The decode step for each batch bucket (decode_graph.py:33-119): :meth:`run` replays the
    smallest bucket that holds the batch and returns None above the largest.  Padded rows write
    and read only the first slot of a scratch page taken from ``cache`` (decode_graph.py:49-53).
    The reference records buckets up to 1024 sequences; this build's GEMMs stream weights for at
    most 64 token rows per launch, so ``max_batch`` is at most 64."""

    def __init__(self, language: LanguageModel, cache: KVCache, *, max_batch: int, max_positions: int,
                 stream: torch.cuda.Stream | None = None):
        if not 1 <= max_batch <= BUCKETS[-1]:
            raise ValueError(f"DecodeGraphs: max_batch must be in [1, {BUCKETS[-1]}]")
        self.language = language
        self.cache = cache
        self.stream = stream or torch.cuda.Stream()
        device = language.weights.lm_head.device
        scratch = cache.allocate(1)
        if scratch is None:
            raise RuntimeError("DecodeGraphs: no free KV page for the scratch page")
        bs = cache.block_size
        self.scratch_block = scratch[0]
        self.scratch_slot = self.scratch_block * bs
        self.buckets = [b for b in BUCKETS if b < max_batch] + [max_batch]
        self.width = -(-max_positions // bs)
        top = self.buckets[-1]

        self.ids = torch.zeros(top, dtype=torch.long, device=device)
        self.positions = torch.zeros(top, dtype=torch.long, device=device)
        self.slots = torch.full((top,), self.scratch_slot, dtype=torch.long, device=device)
        self.seq_lens = torch.ones(top, dtype=torch.int32, device=device)
        self.table = torch.full((top, self.width), self.scratch_block, dtype=torch.int32, device=device)
        self._staging = [(dst, torch.empty_like(dst, device="cpu").pin_memory())
                         for dst in (self.ids, self.positions, self.slots, self.seq_lens, self.table)]
        self._host = [host.numpy() for _, host in self._staging]
        self.buffers = StepBuffers.allocate(language.config, top, 1, self.width * bs, device)
        self.logits = torch.empty(top, language.config.vocab_size, dtype=torch.bfloat16, device=device)

        self._graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor, torch.Tensor]] = {}
        pool = torch.cuda.graph_pool_handle()
        for bucket in reversed(self.buckets):
            self._graphs[bucket] = self._capture(bucket, pool)

    def _forward(self, bucket: int) -> tuple[torch.Tensor, torch.Tensor]:
        batch = DecodeBatch(self.ids[:bucket], self.positions[:bucket], self.slots[:bucket], self.seq_lens[:bucket],
                            self.table[:bucket])
        hidden = self.language.decode(batch, self.cache, self.buffers)
        tokens, logits = lm_head.lm_head_argmax(hidden, self.language.weights.lm_head,
                                                predicted=self.buffers.predicted[:bucket],
                                                logits=self.logits[:bucket], return_logits=True,
                                                workspace=self.buffers.head_workspace)
        return logits, tokens

    def _capture(self, bucket: int, pool) -> tuple[torch.cuda.CUDAGraph, torch.Tensor, torch.Tensor]:
        _warm_up(self.stream, lambda: self._forward(bucket))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=pool, stream=self.stream):
            logits, tokens = self._forward(bucket)
        return graph, logits, tokens

    def run(self, ids: list[int], positions: list[int], slots: list[int], seq_lens: list[int],
            tables: list[list[int]]) -> tuple[torch.Tensor, torch.Tensor] | None:
        """Replays one step; returns ``[n, vocab]`` bf16 logits and ``[n]`` greedy ids (views of the
        bucket's outputs, valid until the next replay), or None when ``n`` exceeds the largest bucket."""
        n = len(ids)
        bucket = next((b for b in self.buckets if b >= n), None)
        if bucket is None:
            return None
        h_ids, h_positions, h_slots, h_seq_lens, h_table = self._host
        h_ids[:n] = ids
        h_ids[n:bucket] = 0
        h_positions[:n] = positions
        h_positions[n:bucket] = 0
        h_slots[:n] = slots
        h_slots[n:bucket] = self.scratch_slot
        h_seq_lens[:n] = seq_lens
        h_seq_lens[n:bucket] = 1
        pack_page_table(h_table[:bucket], tables, self.scratch_block)
        for dst, host in self._staging:
            dst[:bucket].copy_(host[:bucket], non_blocking=True)
        graph, logits, tokens = self._graphs[bucket]
        graph.replay()
        return logits[:n], tokens[:n]


class ExtendGraphs:
    """The verify forward for ``tokens_per_seq`` tokens per sequence, one graph per bucket."""

    def __init__(self, language: LanguageModel, cache: KVCache, *, max_batch: int, tokens_per_seq: int,
                 max_positions: int, scratch_block: int, stream: torch.cuda.Stream | None = None):
        self.language = language
        self.cache = cache
        self.stream = stream or torch.cuda.Stream()
        self.tokens_per_seq = s = tokens_per_seq
        device = language.weights.lm_head.device
        bs = cache.block_size
        self.buckets = [b for b in EXTEND_BUCKETS if b < max_batch] + [max_batch]
        self.width = -(-max_positions // bs)
        self.scratch_block = scratch_block
        top = self.buckets[-1]
        scratch_slots = torch.arange(s, device=device) + scratch_block * bs

        self.ids = torch.zeros(top * s, dtype=torch.long, device=device)
        self.positions = torch.arange(s, device=device).repeat(top)
        self.slots = scratch_slots.repeat(top)
        self.seq_lens = torch.full((top,), s, dtype=torch.int32, device=device)
        self.table = torch.full((top, self.width), scratch_block, dtype=torch.int32, device=device)
        self._scratch_slots = scratch_slots.cpu().numpy()
        self._staging = [(dst, torch.empty_like(dst, device="cpu").pin_memory())
                         for dst in (self.ids, self.positions, self.slots, self.seq_lens, self.table)]
        self._host = [host.numpy() for _, host in self._staging]
        self.buffers = StepBuffers.allocate(language.config, top, s, self.width * bs, device)

        self._graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}
        pool = torch.cuda.graph_pool_handle()
        for bucket in reversed(self.buckets):
            self._graphs[bucket] = self._capture(bucket, pool)

    def _forward(self, bucket: int) -> torch.Tensor:
        s, n = self.tokens_per_seq, bucket * self.tokens_per_seq
        batch = ExtendBatch(self.ids[:n], self.positions[:n], self.slots[:n], self.seq_lens[:bucket],
                            self.table[:bucket], s)
        hidden = self.language.extend(batch, self.cache, self.buffers)
        return self.language.greedy(hidden, self.buffers).view(bucket, s)

    def _capture(self, bucket: int, pool) -> tuple[torch.cuda.CUDAGraph, torch.Tensor]:
        _warm_up(self.stream, lambda: self._forward(bucket))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=pool, stream=self.stream):
            tokens = self._forward(bucket)
        return graph, tokens

    def run(self, ids: list[int], positions: list[int], slots: list[int], seq_lens: list[int],
            tables: list[list[int]]) -> torch.Tensor | None:
        """``ids``/``positions``/``slots`` hold ``len(seq_lens) * tokens_per_seq`` entries, sequence by
        sequence.  Replays once and returns the greedy ids ``[n, tokens_per_seq]`` (a view of the
        bucket's output, valid until the next replay); None when ``n`` exceeds the largest bucket."""
        n = len(seq_lens)
        bucket = next((b for b in self.buckets if b >= n), None)
        if bucket is None:
            return None
        s = self.tokens_per_seq
        real, padded = n * s, bucket * s
        h_ids, h_positions, h_slots, h_seq_lens, h_table = self._host
        h_ids[:real] = ids
        h_ids[real:padded] = 0
        h_positions[:real] = positions
        h_positions[real:padded] = np.tile(np.arange(s), bucket - n)
        h_slots[:real] = slots
        h_slots[real:padded] = np.tile(self._scratch_slots, bucket - n)
        h_seq_lens[:n] = seq_lens
        h_seq_lens[n:bucket] = s
        pack_page_table(h_table[:bucket], tables, self.scratch_block)
        for dst, host in self._staging:
            length = padded if dst.shape[0] == self.ids.shape[0] else bucket
            dst[:length].copy_(host[:length], non_blocking=True)
        graph, tokens = self._graphs[bucket]
        graph.replay()
        return tokens[:n]


class VerifyLoop:
    """The complete device-resident verify step for a fixed batch of ``batch`` sequences."""

    def __init__(self, language: LanguageModel, cache: KVCache, *, batch: int, k: int, max_n: int = 4,
                 history_capacity: int, table_width: int, eos_id: int = -1, device="cuda"):
        self.language, self.cache = language, cache
        self.batch, self.k, self.max_n = batch, k, max_n
        self.tokens_per_seq = s = k + 1
        self.eos_id = eos_id
        i32 = dict(dtype=torch.int32, device=device)
        self.history = torch.zeros(batch, history_capacity, **i32)
        self.history_len = torch.zeros(batch, **i32)
        self.seq_len = torch.zeros(batch, **i32)
        self.block_table = torch.zeros(batch, table_width, **i32)
        self.finished = torch.zeros(batch, **i32)
        self.inputs = speculative.alloc_verify_inputs(batch, k, s, torch.device(device))
        self.buffers = StepBuffers.allocate(language.config, batch, s, table_width * cache.block_size, device)
        self.accepted = speculative.AcceptResult(torch.zeros(batch, **i32), torch.zeros(batch, k + 1, **i32),
                                                 torch.zeros(batch, **i32))
        self.graph: torch.cuda.CUDAGraph | None = None
        self.stream: torch.cuda.Stream | None = None

    def load(self, histories: list[np.ndarray], seq_lens: np.ndarray, block_table: np.ndarray) -> None:
        """Host state in: each sequence's generated ids, its KV length (``seq.length``) and pages."""
        cap = self.history.shape[1]
        hist = np.zeros((self.batch, cap), dtype=np.int32)
        lens = np.zeros(self.batch, dtype=np.int32)
        for b, h in enumerate(histories):
            hist[b, : len(h)] = h
            lens[b] = len(h)
        self.history.copy_(torch.from_numpy(hist))
        self.history_len.copy_(torch.from_numpy(lens))
        self.seq_len.copy_(torch.from_numpy(np.asarray(seq_lens, dtype=np.int32)))
        table = np.zeros(tuple(self.block_table.shape), dtype=np.int32)
        table[:, : block_table.shape[1]] = block_table
        self.block_table.copy_(torch.from_numpy(table))
        self.finished.zero_()

    def step(self) -> None:
        """Enqueue one verify step on the current stream (no host synchronisation)."""
        inp = speculative.propose_verify_inputs(
            self.history, self.history_len, self.k, self.seq_len, self.block_table, self.cache.block_size,
            self.tokens_per_seq, max_n=self.max_n, out=self.inputs,
        )
        batch = ExtendBatch(inp.ids, inp.positions, inp.slots, inp.attn_seq_lens, self.block_table,
                            self.tokens_per_seq)
        hidden = self.language.extend(batch, self.cache, self.buffers)
        predicted = self.language.greedy(hidden, self.buffers)
        speculative.accept_batch(
            inp.draft, inp.draft_len, predicted.view(self.batch, self.tokens_per_seq), seq_len=self.seq_len,
            history=self.history, history_len=self.history_len, eos_id=self.eos_id, finished=self.finished,
            out=self.accepted,
        )

    def _snapshot(self):
        return [t.clone() for t in (self.history, self.history_len, self.seq_len, self.finished)]

    def _restore(self, saved) -> None:
        for dst, src in zip((self.history, self.history_len, self.seq_len, self.finished), saved):
            dst.copy_(src)

    def capture(self, stream: torch.cuda.Stream | None = None) -> None:
        """Warm up twice (state restored afterwards) and capture one step into a graph."""
        self.stream = stream or torch.cuda.Stream()
        saved = self._snapshot()
        _warm_up(self.stream, self.step)
        self._restore(saved)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.step()
        torch.cuda.synchronize()

    def replay(self) -> None:
        assert self.graph is not None, "capture() first"
        self.graph.replay()
