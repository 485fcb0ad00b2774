"""n-gram drafting and greedy acceptance on the GPU: the drop-in for oxr_runtime/speculative.py.

The reference keeps a per-sequence Python dict (speculative.py:15-39) and accepts on the
host after copying the verify step's greedy ids back (engine.py:727-733).  Here both run
as gfx950 kernels over device-resident histories:

- ``propose_batch``: all sequences' drafts in one launch (csrc/ngram.hip).
- ``propose_verify_inputs``: drafting fused with the verify-row assembly of
  engine.py:700-710 (ids, positions, slots, seq_lens), so the step needs no host data.
- ``accept_batch``: longest-prefix acceptance, length rollback and history append for
  all sequences in one launch (csrc/accept.hip).
- ``greedy_accept_batch``: the LM head's greedy ids and ``accept_batch`` on them, with the
  argmax finished inside the acceptance launch.

``NgramProposer`` and ``accept`` keep the reference's list-based signatures for callers
that hold Python lists; they run the same kernels on a batch of one.
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import NamedTuple

import torch

from . import _lib
from .gemm import PackedWeight

_MAX_N = 4  # speculative.py:12


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("speculative: no GPU visible; this build has no CPU path")
    return torch.device("cuda", torch.cuda.current_device())


def _check_int32(name: str, t: torch.Tensor, dims: int) -> None:
    _lib.require(t.dtype == torch.int32 and t.dim() == dims, f"{name} must be int32 with {dims} dims")
    _lib.require(t.is_contiguous(), f"{name} must be contiguous")


def propose_batch(
    history: torch.Tensor, history_len: torch.Tensor, k: int, *, max_n: int = _MAX_N,
    k_limit: torch.Tensor | None = None, index_len: torch.Tensor | None = None,
    draft: torch.Tensor | None = None, draft_len: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Drafts for every sequence: ``history`` int32 ``[B, capacity]`` with ``history_len[b]`` valid
    tokens.  Returns (``draft`` int32 ``[B, k]`` zero-padded, ``draft_len`` int32 ``[B]``); row b is
    ``NgramProposer(h).propose(h, min(k, k_limit[b]))`` of the reference for ``h = history[b, :len]``."""
    device = _lib.require_gpu(history, history_len, k_limit, index_len, name="propose_batch")
    _check_int32("history", history, 2)
    _check_int32("history_len", history_len, 1)
    b = history.shape[0]
    _lib.require(history_len.shape[0] == b, "history_len must be [B]")
    for name, t in (("k_limit", k_limit), ("index_len", index_len)):
        if t is not None:
            _check_int32(name, t, 1)
            _lib.require(t.shape[0] == b, f"{name} must be [B]")
    if draft is None:
        draft = torch.empty(b, k, dtype=torch.int32, device=device)
    if draft_len is None:
        draft_len = torch.empty(b, dtype=torch.int32, device=device)
    _lib.require(draft.shape == (b, k) and draft.dtype == torch.int32 and draft.is_contiguous(), "draft must be int32 [B, k]")
    _check_int32("draft_len", draft_len, 1)
    _lib.call(
        "oxr_ngram_propose", history.data_ptr(), history.stride(0), history_len.data_ptr(), _lib.ptr(index_len), b,
        max_n, k, _lib.ptr(k_limit), draft.data_ptr(), draft_len.data_ptr(), _lib.stream(device),
    )
    return draft, draft_len


class VerifyInputs(NamedTuple):
    draft: torch.Tensor          # int32 [B, k]
    draft_len: torch.Tensor      # int32 [B]
    ids: torch.Tensor            # int64 [B * S]
    positions: torch.Tensor      # int64 [B * S]
    slots: torch.Tensor          # int64 [B * S]
    attn_seq_lens: torch.Tensor  # int32 [B]


def alloc_verify_inputs(batch: int, k: int, tokens_per_seq: int, device: torch.device) -> VerifyInputs:
    n = batch * tokens_per_seq
    return VerifyInputs(
        torch.zeros(batch, k, dtype=torch.int32, device=device), torch.zeros(batch, dtype=torch.int32, device=device),
        torch.zeros(n, dtype=torch.int64, device=device), torch.zeros(n, dtype=torch.int64, device=device),
        torch.zeros(n, dtype=torch.int64, device=device), torch.zeros(batch, dtype=torch.int32, device=device),
    )


def propose_verify_inputs(
    history: torch.Tensor, history_len: torch.Tensor, k: int, seq_len: torch.Tensor, block_table: torch.Tensor,
    block_size: int, tokens_per_seq: int, *, max_n: int = _MAX_N, k_limit: torch.Tensor | None = None,
    max_tokens: torch.Tensor | None = None, max_positions: int = 0, out: VerifyInputs | None = None,
) -> VerifyInputs:
    """Drafting plus the verify rows of engine.py:700-710, all on the GPU.  ``seq_len`` is each
    sequence's KV length before the step (the reference's ``seq.length``).  Drafts are capped by
    the room engine.py:683-684 leaves: ``max_tokens[b] - len(history) - 1`` (when given) and
    ``max_positions - seq_len - 1`` (when > 0).  Negative block-table entries (pages not
    allocated) give slot -1: that row's K/V is not stored."""
    device = _lib.require_gpu(history, history_len, seq_len, block_table, k_limit, max_tokens,
                              name="propose_verify_inputs")
    _check_int32("history", history, 2)
    _check_int32("history_len", history_len, 1)
    _check_int32("seq_len", seq_len, 1)
    _check_int32("block_table", block_table, 2)
    b = history.shape[0]
    _lib.require(tokens_per_seq >= k + 1, "tokens_per_seq must be at least k + 1")
    _lib.require(block_table.shape[0] >= b and history_len.shape[0] == b and seq_len.shape[0] == b, "batch sizes differ")
    if max_tokens is not None:
        _check_int32("max_tokens", max_tokens, 1)
        _lib.require(max_tokens.shape[0] == b, "max_tokens must be [B]")
    if out is None:
        out = alloc_verify_inputs(b, k, tokens_per_seq, device)
    _lib.call(
        "oxr_propose_verify_inputs", history.data_ptr(), history.stride(0), history_len.data_ptr(), b, max_n, k,
        _lib.ptr(k_limit), seq_len.data_ptr(), block_table.data_ptr(), block_table.stride(0), block_size,
        tokens_per_seq, _lib.ptr(max_tokens), int(max_positions), out.draft.data_ptr(), out.draft_len.data_ptr(),
        out.ids.data_ptr(), out.positions.data_ptr(), out.slots.data_ptr(), out.attn_seq_lens.data_ptr(),
        _lib.stream(device),
    )
    return out


class AcceptResult(NamedTuple):
    accepted: torch.Tensor       # int32 [B]: drafts accepted (a)
    committed: torch.Tensor      # int32 [B, k+1]: predicted[:a+1], rest -1
    num_committed: torch.Tensor  # int32 [B]: a + 1


def _accept_args(draft, draft_len, s, seq_len, history, history_len, max_tokens, finished, out, device):
    """Checks shared by the acceptance entry points; the output tensors (``out`` or new ones)."""
    _check_int32("draft", draft, 2)
    _check_int32("draft_len", draft_len, 1)
    b, k = draft.shape
    for name, t in (("seq_len", seq_len), ("history_len", history_len), ("max_tokens", max_tokens),
                    ("finished", finished)):
        if t is not None:
            _check_int32(name, t, 1)
            _lib.require(t.shape[0] == b, f"{name} must be [B]")
    if history is not None:
        _check_int32("history", history, 2)
        _lib.require(history_len is not None, "history needs history_len")
    if out is None:
        out = AcceptResult(torch.empty(b, dtype=torch.int32, device=device),
                           torch.empty(b, k + 1, dtype=torch.int32, device=device),
                           torch.empty(b, dtype=torch.int32, device=device))
    return out


def accept_batch(
    draft: torch.Tensor, draft_len: torch.Tensor, predicted: torch.Tensor, *, seq_len: torch.Tensor | None = None,
    history: torch.Tensor | None = None, history_len: torch.Tensor | None = None, eos_id: int = -1,
    max_tokens: torch.Tensor | None = None, finished: torch.Tensor | None = None, out: AcceptResult | None = None,
) -> AcceptResult:
    """speculative.accept for every sequence plus the engine's rollback (engine.py:729-737):
    ``seq_len += a + 1`` and the committed ids appended to ``history`` (stopping at ``eos_id`` or
    ``max_tokens``, reported in ``finished``).  ``predicted`` is the step's int64 ``[B, S]`` greedy ids."""
    device = _lib.require_gpu(draft, draft_len, predicted, seq_len, history, history_len, max_tokens, finished,
                              name="accept_batch")
    b, k = draft.shape
    _lib.require(predicted.dtype == torch.int64 and predicted.dim() == 2 and predicted.shape[0] == b
                 and predicted.is_contiguous(), "predicted must be contiguous int64 [B, S]")
    s = predicted.shape[1]
    out = _accept_args(draft, draft_len, s, seq_len, history, history_len, max_tokens, finished, out, device)
    _lib.call(
        "oxr_accept", draft.data_ptr(), draft_len.data_ptr(), k, predicted.data_ptr(), s, b, int(eos_id),
        _lib.ptr(max_tokens), out.accepted.data_ptr(), out.committed.data_ptr(), out.num_committed.data_ptr(),
        _lib.ptr(seq_len), _lib.ptr(history), history.stride(0) if history is not None else 0, _lib.ptr(history_len),
        _lib.ptr(finished), _lib.stream(device),
    )
    return out


def greedy_accept_batch(
    hidden: torch.Tensor, head_weight: PackedWeight, draft: torch.Tensor, draft_len: torch.Tensor, *,
    predicted: torch.Tensor, workspace: torch.Tensor, seq_len: torch.Tensor | None = None,
    history: torch.Tensor | None = None, history_len: torch.Tensor | None = None, eos_id: int = -1,
    max_tokens: torch.Tensor | None = None, finished: torch.Tensor | None = None, out: AcceptResult | None = None,
) -> AcceptResult:
    """The verify step's tail in two launches (``oxr_lm_head_accept_packed``): the greedy ids of
    ``hidden`` (bf16 ``[B * S, hidden]``) under the packed LM head ``head_weight`` into ``predicted`` (int64
    ``[B, S]``; language.py:213-214, decode_graph.py:167), then :func:`accept_batch` on them, with
    the argmax's last reduction done by the acceptance launch.  Same results as
    ``lm_head.lm_head_argmax`` followed by :func:`accept_batch`.  ``workspace``: at least
    ``lm_head.workspace_bytes(B * S, vocab)`` bytes."""
    device = _lib.require_gpu(hidden, head_weight.data, draft, draft_len, predicted, workspace, seq_len, history,
                              history_len, max_tokens, finished, name="greedy_accept_batch")
    b, k = draft.shape
    _lib.require(predicted.dtype == torch.int64 and predicted.dim() == 2 and predicted.shape[0] == b
                 and predicted.is_contiguous(), "predicted must be contiguous int64 [B, S]")
    s = predicted.shape[1]
    _lib.require(hidden.dtype == torch.bfloat16 and hidden.dim() == 2 and hidden.shape[0] == b * s
                 and hidden.stride(1) == 1 and hidden.shape[1] == head_weight.shape[1],
                 "hidden must be bf16 [B * S, hidden] with contiguous rows")
    _lib.require(hidden.stride(0) == hidden.shape[1], "hidden rows must be packed back to back")
    out = _accept_args(draft, draft_len, s, seq_len, history, history_len, max_tokens, finished, out, device)
    _lib.call(
        "oxr_lm_head_accept_packed", hidden.data_ptr(), b * s, head_weight.data.data_ptr(), hidden.shape[1],
        head_weight.shape[0], workspace.data_ptr(), workspace.numel() * workspace.element_size(), predicted.data_ptr(),
        draft.data_ptr(), draft_len.data_ptr(), k, s, b, int(eos_id), _lib.ptr(max_tokens), out.accepted.data_ptr(),
        out.committed.data_ptr(), out.num_committed.data_ptr(), _lib.ptr(seq_len), _lib.ptr(history),
        history.stride(0) if history is not None else 0, _lib.ptr(history_len), _lib.ptr(finished),
        _lib.stream(device),
    )
    return out


class NgramProposer:
    """speculative.py:15-39 with the same methods, over a device-resident copy of the history.

    The history is mirrored on the GPU append-only: ``propose``/``extend`` upload only tokens
    past the mirrored length (a shorter list re-uploads everything).  The index covers positions
    up to the length at the last ``__init__``/``extend``, as the reference's dict does.  One call
    of ``propose`` costs one host-to-device copy (the new tokens and the two lengths travel in one
    pinned buffer) and one device-to-host read (the draft and its length together)."""

    def __init__(self, tokens: Sequence[int], *, max_n: int = _MAX_N):
        self.max_n = max_n
        self._device = _device()
        self._buf = torch.zeros(max(64, 2 * len(tokens)), dtype=torch.int32, device=self._device)
        self._mirrored = 0
        self._indexed = len(tokens)
        self._k = -1
        self._stage_host = torch.zeros(0, dtype=torch.int32)
        self._copied: torch.cuda.Event | None = None  # the last upload from the staging buffer
        self._sync(tokens)

    def _sync(self, tokens: Sequence[int]) -> None:
        """Mirror ``tokens`` and stage [len, indexed] for the next launch, in one upload."""
        n = len(tokens)
        if n < self._mirrored:
            self._mirrored = 0
        if n > self._buf.numel():
            grown = torch.zeros(2 * n, dtype=torch.int32, device=self._device)
            grown[: self._mirrored] = self._buf[: self._mirrored]
            self._buf = grown
        new = n - self._mirrored
        if self._copied is not None:
            self._copied.synchronize()  # the staging buffer is rewritten below: its last upload must be done
        if self._stage_host.numel() < new + 2:
            self._stage_host = torch.empty(max(2 * (new + 2), 64), dtype=torch.int32).pin_memory()
            self._stage_dev = torch.empty(self._stage_host.numel(), dtype=torch.int32, device=self._device)
        host = self._stage_host.numpy()
        host[0], host[1] = n, self._indexed
        host[2 : 2 + new] = tokens[self._mirrored :]
        self._stage_dev[: new + 2].copy_(self._stage_host[: new + 2], non_blocking=True)
        self._copied = torch.cuda.Event()
        self._copied.record()
        if new:
            self._buf[self._mirrored : n].copy_(self._stage_dev[2 : 2 + new])
        self._mirrored = n

    def extend(self, tokens: Sequence[int], old_length: int) -> None:
        """``tokens`` from ``old_length`` on are new; index them (speculative.py:28-31).

        The reference adds positions ``[max(old_length, 1), len(tokens))`` to its dict.  The device
        index is a prefix of the history (every position below ``index_len``), which is the same
        set whenever ``old_length`` does not skip past what is already indexed: then the union is
        ``[1, len(tokens))`` and each n-gram's latest position is its maximum, as in the dict.  An
        ``old_length`` beyond the indexed length would leave a gap the prefix cannot express, so it
        raises ``ValueError`` (the engine always passes the previous length, engine.py:677-681)."""
        if old_length > self._indexed:
            raise ValueError(f"extend: old_length {old_length} would leave positions [{self._indexed}, {old_length}) "
                             "unindexed; the device index covers a prefix of the history")
        self._indexed = max(self._indexed, len(tokens))
        self._sync(tokens)

    def propose(self, tokens: Sequence[int], k: int) -> list[int]:
        """Up to ``k`` ids following the latest earlier occurrence of the longest matching suffix;
        ``[]`` when nothing matches (speculative.py:33-39)."""
        self._sync(tokens)
        n = len(tokens)
        k = max(k, 0)
        if k != self._k:
            self._out = torch.zeros(k + 1, dtype=torch.int32, device=self._device)  # [len, draft...]
            self._k = k
        hist = self._buf[:n].view(1, n) if n else self._buf[:1].view(1, 1)
        propose_batch(hist, self._stage_dev[0:1], k, max_n=self.max_n, index_len=self._stage_dev[1:2],
                      draft=self._out[1:].view(1, k), draft_len=self._out[0:1])
        out = self._out.tolist()  # the one synchronising read
        return out[1 : 1 + out[0]]


def accept(draft: Sequence[int], predicted: Sequence[int]) -> list[int]:
    """``predicted[j]`` is the model's choice after the previous token and ``draft[:j]``
    (``len(predicted) == len(draft) + 1``).  Returns the matching prefix of ``draft`` plus the model's
    next choice (speculative.py:42-48).  One host-to-device copy (draft and predicted ids in one
    buffer) and one device-to-host read."""
    device = _device()
    k = len(draft)
    _lib.require(len(predicted) >= k + 1, "predicted must hold len(draft) + 1 ids")
    staged = torch.tensor([k, *draft, *predicted[: k + 1]], dtype=torch.int64).pin_memory()
    dev = staged.to(device, non_blocking=True)
    d = dev[1 : 1 + k].to(torch.int32).view(1, k) if k else torch.zeros(1, 1, dtype=torch.int32, device=device)
    dl = dev[0:1].to(torch.int32)
    p = dev[1 + k : 2 + 2 * k].view(1, k + 1)
    res = accept_batch(d, dl, p)
    a = int(res.accepted.item())  # the one synchronising read
    return list(draft[:a]) + [int(predicted[a])]
