"""HIP-graph capture and replay of the decode and speculative verify steps.

Three entry points:

- :class:`DecodeGraphs`: the one-token decode step (the interface of
  oxr_runtime/decode_graph.py:33-119): host lists in, ``(logits, greedy ids)`` out.
- :class:`ExtendGraphs`: the verify forward for a fixed number S of tokens per sequence (the
  interface of oxr_runtime/decode_graph.py:122-205): host lists in, greedy ids ``[n, S]`` out.
- :class:`VerifyLoop`: the whole speculative step with nothing on the host -- drafting and row
  assembly (engine.py:674-710), the forward, LM head + argmax, acceptance and length/history
  rollback (engine.py:729-737) -- in one graph replayed back to back.  Histories, lengths and
  block tables stay in device memory; each replay drafts from what the previous one committed.

The first two share one runner, :class:`_BucketedStep`.  A step's inputs travel as one compact
int64 record (:class:`_StepRecord`: the real sequences' rows and their page lists, no padding)
in one host-to-device copy; the first node of every captured graph expands it on the device
(``oxr_unpack_step_inputs``) into the bucket's fixed tensors, padding the bucket with rows that
write and read only the first S slots of a scratch page, as the reference's padded rows do
(decode_graph.py:188-197).  Outputs are views of the bucket's buffers, valid until the next replay.

Graphs are captured on an ordinary stream (default priority); the reference captures on a
high-priority stream (decode_graph.py:14-17), and stream priorities are avoided on this platform.
"""

from __future__ import annotations

import functools
import gc
import itertools
from collections.abc import Callable, Sequence

import numpy as np
import torch

from . import _lib, gemm, lm_head, speculative
from .kv_cache import KVCache
from .language import DecodeBatch, ExtendBatch, LanguageModel, StepBuffers

# Batch buckets: the reference's lists (decode_graph.py:30, 122), kept up to the largest token-row
# count one forward takes (gemm.MAX_ROWS).
BUCKETS = tuple(b for b in (1, 2, 4, 8, 16, 32, 64, 128, 192, 256, 384, 512, 768, 1024) if b <= gemm.MAX_ROWS)
EXTEND_BUCKETS = (1, 2, 4, 8)


def _collect_before_capture() -> None:
    """Free unreachable objects now: a graph freed by the garbage collector while a stream is
    capturing would end the process (HIP refuses to destroy a graph during a capture)."""
    gc.collect()


class _StepRecord:
    """One step's inputs for up to ``capacity`` sequences of ``s`` rows: a pinned int64 record and
    its device twin, laid out as csrc/step_inputs.hip expects.  :meth:`write` fills the host side
    and enqueues one copy of the used words on the current stream.  The host side is reused on the
    next :meth:`write`: as with the reference's staging buffers, the caller reads a replay's
    outputs (which waits for it, and so for its copy) before the next step."""

    def __init__(self, capacity: int, s: int, width: int, device: torch.device):
        self.capacity, self.s, self.width = capacity, s, width
        words = int(_lib.lib().oxr_step_record_words(capacity, s, width))
        self.host = torch.zeros(words, dtype=torch.int64).pin_memory()
        self.device = torch.zeros(words, dtype=torch.int64, device=device)
        t = capacity * s
        a = self.host.numpy()
        self._head = a[:2]
        self._ids, self._positions, self._slots = a[2 : 2 + t], a[2 + t : 2 + 2 * t], a[2 + 2 * t : 2 + 3 * t]
        self._seq_lens = a[2 + 3 * t : 2 + 3 * t + capacity]
        self._offsets = a[2 + 3 * t + capacity : 2 + 3 * t + 2 * capacity + 1]
        self._pages_at = 2 + 3 * t + 2 * capacity + 1
        self._pages = a[self._pages_at :]

    def write(self, ids: Sequence[int], positions: Sequence[int], slots: Sequence[int], seq_lens: Sequence[int],
              tables: Sequence[Sequence[int]]) -> None:
        n, rows = len(seq_lens), len(seq_lens) * self.s
        _lib.require(n <= self.capacity, f"{n} sequences, the record holds {self.capacity}")
        _lib.require(len(ids) == rows and len(positions) == rows and len(slots) == rows,
                     f"ids, positions and slots must hold {rows} entries ({n} sequences x {self.s})")
        _lib.require(len(tables) == n, "one page list per sequence")
        counts = np.fromiter(map(len, tables), dtype=np.int64, count=n)
        _lib.require(not (counts > self.width).any(), f"a page list is longer than the table width {self.width}")
        self._offsets[0] = 0
        np.cumsum(counts, out=self._offsets[1 : n + 1])
        total = int(self._offsets[n])
        self._pages[:total] = np.fromiter(itertools.chain.from_iterable(tables), dtype=np.int64, count=total)
        self._ids[:rows], self._positions[:rows], self._slots[:rows] = ids, positions, slots
        self._seq_lens[:n] = seq_lens
        self._head[:] = (n, total)
        used = self._pages_at + total
        self.device[:used].copy_(self.host[:used], non_blocking=True)


class _BucketedStep:
    """A step of ``s`` rows per sequence, one HIP graph per batch bucket.

    ``forward(step, bucket)`` enqueues the step on the fixed tensors ``ids``/``positions``/``slots``
    (``[top * s]``), ``seq_lens`` (``[top]``) and ``table`` (``[top, width]``) restricted to the
    bucket, and returns its outputs.  Each graph starts with the expansion of the device record
    into those tensors.  Buckets are captured largest first, so the smaller ones reuse its pool."""

    def __init__(self, cache: KVCache, buckets: list[int], s: int, width: int, scratch_block: int, device,
                 stream: torch.cuda.Stream | None, forward: Callable[["_BucketedStep", int], object]):
        self.cache, self.buckets, self.s, self.width = cache, buckets, s, width
        self.scratch_block = scratch_block
        self.stream = stream or torch.cuda.Stream()
        top = buckets[-1]
        self.ids = torch.zeros(top * s, dtype=torch.int64, device=device)
        self.positions = torch.zeros(top * s, dtype=torch.int64, device=device)
        self.slots = torch.zeros(top * s, dtype=torch.int64, device=device)
        self.seq_lens = torch.zeros(top, dtype=torch.int32, device=device)
        self.table = torch.zeros(top, width, dtype=torch.int32, device=device)
        self.record = _StepRecord(top, s, width, device)
        self._forward = forward
        self._graphs: dict[int, tuple[torch.cuda.CUDAGraph, object]] = {}
        pool = torch.cuda.graph_pool_handle()
        for bucket in reversed(buckets):
            self._graphs[bucket] = self._capture(bucket, pool)

    def _body(self, bucket: int):
        _lib.call("oxr_unpack_step_inputs", self.record.device.data_ptr(), self.record.capacity, bucket, self.s,
                  self.width, self.scratch_block, self.cache.block_size, self.ids.data_ptr(),
                  self.positions.data_ptr(), self.slots.data_ptr(), self.seq_lens.data_ptr(), self.table.data_ptr(),
                  _lib.stream(self.ids.device))
        return self._forward(self, bucket)

    def _capture(self, bucket: int, pool) -> tuple[torch.cuda.CUDAGraph, object]:
        # One eager pass on the capture stream first (one-time launch set-up happens outside the
        # capture), with the record still empty: every row is a scratch row.
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self.stream):
            self._body(bucket)
        torch.cuda.current_stream().wait_stream(self.stream)
        _collect_before_capture()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=pool, stream=self.stream):
            out = self._body(bucket)
        return graph, out

    def bucket_for(self, n: int) -> int | None:
        return next((b for b in self.buckets if b >= n), None)

    def graph(self, bucket: int) -> torch.cuda.CUDAGraph:
        return self._graphs[bucket][0]

    def replay(self, ids, positions, slots, seq_lens, tables):
        bucket = self.bucket_for(len(seq_lens))
        if bucket is None:
            return None
        self.record.write(ids, positions, slots, seq_lens, tables)
        graph, out = self._graphs[bucket]
        graph.replay()
        return out


def _decode_forward(language: LanguageModel, cache: KVCache, buffers: StepBuffers, logits: torch.Tensor,
                    st: _BucketedStep, bucket: int) -> tuple[torch.Tensor, torch.Tensor]:
    batch = DecodeBatch(None, st.positions[:bucket], st.slots[:bucket], st.seq_lens[:bucket], st.table[:bucket],
                        ids=st.ids[:bucket])
    hidden = language.decode(batch, cache, buffers)
    tokens, out = lm_head.lm_head_argmax(hidden, language.weights.lm_head, predicted=buffers.predicted[:bucket],
                                         logits=logits[:bucket], return_logits=True,
                                         workspace=buffers.head_workspace)
    return out, tokens


def _extend_forward(language: LanguageModel, cache: KVCache, buffers: StepBuffers, st: _BucketedStep,
                    bucket: int) -> torch.Tensor:
    s = st.s
    batch = ExtendBatch(None, st.positions[: bucket * s], st.slots[: bucket * s], st.seq_lens[:bucket],
                        st.table[:bucket], s, ids=st.ids[: bucket * s])
    hidden = language.extend(batch, cache, buffers)
    return language.greedy(hidden, buffers).view(bucket, s)


class DecodeGraphs:
    """The decode step per batch bucket (interface of decode_graph.py:33-119): :meth:`run` replays
    the smallest bucket that holds the batch and returns None above the largest.  Padded rows write
    and read only the first slot of a scratch page taken from ``cache`` (decode_graph.py:49-53)."""

    def __init__(self, language: LanguageModel, cache: KVCache, *, max_batch: int, max_positions: int,
                 stream: torch.cuda.Stream | None = None):
        if not 1 <= max_batch <= BUCKETS[-1]:
            raise ValueError(f"DecodeGraphs: max_batch must be in [1, {BUCKETS[-1]}]")
        self.language, self.cache = language, cache
        scratch = cache.allocate(1)
        if scratch is None:
            raise RuntimeError("DecodeGraphs: no free KV page for the scratch page")
        self.scratch_block = scratch[0]
        self.scratch_slot = self.scratch_block * cache.block_size
        self.buckets = [b for b in BUCKETS if b < max_batch] + [max_batch]
        self.width = -(-max_positions // cache.block_size)
        device = language.weights.lm_head.device
        top = self.buckets[-1]
        self.buffers = StepBuffers.allocate(language.config, top, 1, self.width * cache.block_size, device)
        self.logits = torch.empty(top, language.config.vocab_size, dtype=torch.bfloat16, device=device)
        # (The forward is bound to the parts it uses, not to self: no reference cycle, so the graphs
        # are freed when the runner is dropped rather than by a later garbage collection.)
        forward = functools.partial(_decode_forward, language, cache, self.buffers, self.logits)
        self._step = _BucketedStep(cache, self.buckets, 1, self.width, self.scratch_block, device, stream, forward)
        self.stream = self._step.stream

    def graph(self, bucket: int) -> torch.cuda.CUDAGraph:
        return self._step.graph(bucket)

    def run(self, ids: list[int], positions: list[int], slots: list[int], seq_lens: list[int],
            tables: list[list[int]]) -> tuple[torch.Tensor, torch.Tensor] | None:
        """One step: ``[n, vocab]`` bf16 logits and ``[n]`` greedy ids, or None above the largest bucket."""
        out = self._step.replay(ids, positions, slots, seq_lens, tables)
        if out is None:
            return None
        n = len(ids)
        return out[0][:n], out[1][:n]


class ExtendGraphs:
    """The verify forward for ``tokens_per_seq`` tokens per sequence, one graph per bucket
    (interface of decode_graph.py:125-205, buckets 1, 2, 4, 8 and ``max_batch``).  Padded rows
    write the first S slots of ``scratch_block`` and attend only to them."""

    def __init__(self, language: LanguageModel, cache: KVCache, *, max_batch: int, tokens_per_seq: int,
                 max_positions: int, scratch_block: int, stream: torch.cuda.Stream | None = None):
        if max_batch < 1 or max_batch * tokens_per_seq > gemm.MAX_ROWS:
            raise ValueError(f"ExtendGraphs: max_batch * tokens_per_seq must be in [1, {gemm.MAX_ROWS}]")
        self.language, self.cache = language, cache
        self.tokens_per_seq = tokens_per_seq
        self.scratch_block = scratch_block
        self.buckets = [b for b in EXTEND_BUCKETS if b < max_batch] + [max_batch]
        self.width = -(-max_positions // cache.block_size)
        device = language.weights.lm_head.device
        self.buffers = StepBuffers.allocate(language.config, self.buckets[-1], tokens_per_seq,
                                            self.width * cache.block_size, device)
        forward = functools.partial(_extend_forward, language, cache, self.buffers)
        self._step = _BucketedStep(cache, self.buckets, tokens_per_seq, self.width, scratch_block, device, stream,
                                   forward)
        self.stream = self._step.stream

    def graph(self, bucket: int) -> torch.cuda.CUDAGraph:
        return self._step.graph(bucket)

    def run(self, ids: list[int], positions: list[int], slots: list[int], seq_lens: list[int],
            tables: list[list[int]]) -> torch.Tensor | None:
        """``ids``/``positions``/``slots`` hold ``len(seq_lens) * tokens_per_seq`` entries, sequence by
        sequence.  Returns the greedy ids ``[n, tokens_per_seq]``, or None above the largest bucket."""
        tokens = self._step.replay(ids, positions, slots, seq_lens, tables)
        return None if tokens is None else tokens[: len(seq_lens)]


# VerifyLoop plans attention pieces (balance=None) for batches of at least BALANCE_MIN_BATCH sequences
# whose longest loaded context is over BALANCE_RATIO times the shortest.  Measured on MI355X at
# contexts U[1k, 16k]: B = 8 and 16 steps 1.6-1.9% faster, B = 4 even, B = 1 5% slower (a plan adds a
# launch per step and a dependent load per attention launch).
BALANCE_RATIO = 1.5
BALANCE_MIN_BATCH = 8


class VerifyLoop:
    """The complete device-resident verify step for a fixed batch of ``batch`` sequences.

    Drafts are capped by the room engine.py:683-684 leaves (``max_tokens`` per sequence, when
    given, and ``max_positions``, by default the table's span).  The loop cannot allocate KV pages:
    table entries past the pages given to :meth:`load` are -1 (their rows get slot -1 and are not
    stored), and :meth:`replay` refuses a step once some sequence could need a position past its
    pages (each step advances a sequence by at most S positions)."""

    def __init__(self, language: LanguageModel, cache: KVCache, *, batch: int, k: int, max_n: int = 4,
                 history_capacity: int, table_width: int, eos_id: int = -1, max_positions: int | None = None,
                 balance: bool | None = None, device="cuda"):
        self.language, self.cache = language, cache
        # Attention context pieces from a per-step plan (attention.build_plan): on, off, or (None)
        # decided at the first load() before capture (see BALANCE_RATIO).
        self.balance = balance
        self.batch, self.k, self.max_n = batch, k, max_n
        self.tokens_per_seq = s = k + 1
        if batch * s > gemm.MAX_ROWS:
            raise ValueError(f"VerifyLoop: batch * (k + 1) must be at most {gemm.MAX_ROWS}")
        self.eos_id = eos_id
        self.max_positions = table_width * cache.block_size if max_positions is None else max_positions
        i32 = dict(dtype=torch.int32, device=device)
        self.history = torch.zeros(batch, history_capacity, **i32)
        self.history_len = torch.zeros(batch, **i32)
        self.seq_len = torch.zeros(batch, **i32)
        self.block_table = torch.full((batch, table_width), -1, **i32)
        self.finished = torch.zeros(batch, **i32)
        self.max_tokens: torch.Tensor | None = None
        self.inputs = speculative.alloc_verify_inputs(batch, k, s, torch.device(device))
        self.buffers = StepBuffers.allocate(language.config, batch, s, table_width * cache.block_size, device)
        if balance:
            self.buffers.enable_plan(language.config, s)
        self.accepted = speculative.AcceptResult(torch.zeros(batch, **i32), torch.zeros(batch, k + 1, **i32),
                                                 torch.zeros(batch, **i32))
        self.graph: torch.cuda.CUDAGraph | None = None
        self.stream: torch.cuda.Stream | None = None
        self.steps_left = 0

    def load(self, histories: list[np.ndarray], seq_lens: np.ndarray, block_table: np.ndarray, *,
             max_tokens: Sequence[int] | None = None) -> None:
        """Host state in: each sequence's generated ids, its KV length (``seq.length``), its pages
        (row b of ``block_table``; negative entries or columns past it: none) and, optionally, its
        ``max_tokens``.  Call before :meth:`capture` when ``max_tokens`` is used."""
        b_, cap = self.batch, self.history.shape[1]
        hist = np.zeros((b_, cap), dtype=np.int32)
        lens = np.zeros(b_, dtype=np.int32)
        for b, h in enumerate(histories):
            _lib.require(len(h) <= cap, "history longer than history_capacity")
            hist[b, : len(h)] = h
            lens[b] = len(h)
        seq = np.asarray(seq_lens, dtype=np.int32)
        width = self.block_table.shape[1]
        block_table = np.asarray(block_table, dtype=np.int32)
        _lib.require(block_table.shape[1] <= width, "block_table wider than table_width")
        table = np.full((b_, width), -1, dtype=np.int32)
        table[:, : block_table.shape[1]] = block_table
        pages = np.cumprod(table >= 0, axis=1).sum(axis=1)  # leading allocated pages
        room = pages * self.cache.block_size - seq
        self.steps_left = int(max(room.min(), 0) // self.tokens_per_seq)
        if self.balance is None and self.graph is None:
            real = seq[: len(histories)] if len(histories) else seq
            if len(real) >= BALANCE_MIN_BATCH and real.max() > BALANCE_RATIO * max(int(real.min()), 1):
                self.buffers.enable_plan(self.language.config, self.tokens_per_seq)
            else:
                self.buffers.balanced = False
        self.history.copy_(torch.from_numpy(hist))
        self.history_len.copy_(torch.from_numpy(lens))
        self.seq_len.copy_(torch.from_numpy(seq))
        self.block_table.copy_(torch.from_numpy(table))
        self.finished.zero_()
        if max_tokens is not None:
            if self.max_tokens is None:
                _lib.require(self.graph is None, "max_tokens must be given before capture()")
                self.max_tokens = torch.zeros(b_, dtype=torch.int32, device=self.history.device)
            self.max_tokens.copy_(torch.tensor(list(max_tokens), dtype=torch.int32))

    def step(self) -> None:
        """Enqueue one verify step on the current stream (no host synchronisation)."""
        inp = speculative.propose_verify_inputs(
            self.history, self.history_len, self.k, self.seq_len, self.block_table, self.cache.block_size,
            self.tokens_per_seq, max_n=self.max_n, max_tokens=self.max_tokens, max_positions=self.max_positions,
            out=self.inputs,
        )
        batch = ExtendBatch(None, inp.positions, inp.slots, inp.attn_seq_lens, self.block_table,
                            self.tokens_per_seq, ids=inp.ids)
        hidden = self.language.extend(batch, self.cache, self.buffers)
        state = dict(seq_len=self.seq_len, history=self.history, history_len=self.history_len, eos_id=self.eos_id,
                     max_tokens=self.max_tokens, finished=self.finished, out=self.accepted)
        head = self.language.weights.lm_head
        if isinstance(head, gemm.PackedWeight):  # the argmax finished inside the acceptance launch
            predicted = self.buffers.predicted[: self.batch * self.tokens_per_seq]
            speculative.greedy_accept_batch(hidden, head, inp.draft, inp.draft_len,
                                            predicted=predicted.view(self.batch, self.tokens_per_seq),
                                            workspace=self.buffers.head_workspace, **state)
        else:
            predicted = self.language.greedy(hidden, self.buffers)
            speculative.accept_batch(inp.draft, inp.draft_len, predicted.view(self.batch, self.tokens_per_seq),
                                     **state)

    def capture(self, stream: torch.cuda.Stream | None = None) -> None:
        """One eager step on the capture stream (state restored afterwards), then the step captured."""
        self.stream = stream or torch.cuda.Stream()
        state = (self.history, self.history_len, self.seq_len, self.finished)
        saved = [t.clone() for t in state]
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self.stream):
            self.step()
        torch.cuda.current_stream().wait_stream(self.stream)
        for dst, src in zip(state, saved):
            dst.copy_(src)
        torch.cuda.synchronize()
        _collect_before_capture()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.step()
        torch.cuda.synchronize()

    def replay(self) -> None:
        if self.graph is None:
            raise RuntimeError("VerifyLoop.replay: capture() first")
        if self.steps_left <= 0:
            raise RuntimeError("VerifyLoop.replay: a sequence could run past its KV pages; load() more pages")
        self.steps_left -= 1
        self.graph.replay()
