"""LM head with fused vocab-wide argmax (csrc/gemm.hip), replacing ``LanguageModel.logits``
(language.py:213-214) followed by ``argmax(dim=-1)`` (decode_graph.py:167, engine.py:726).

The logits are computed tile by tile in fp32, rounded to bf16 (as the reference's bf16
``nn.Linear`` output) and reduced to the first index of the largest value without writing
them out, unless the caller asks for them."""

from __future__ import annotations

import torch

from . import _lib
from .gemm import PackedWeight, Weight

MAX_ROWS = 64          # token rows per launch with a row-major weight
MAX_ROWS_PACKED = 256  # with a packed weight (up to 256 rows read the weight once)


def workspace_bytes(rows: int, vocab: int) -> int:
    """Workspace for ``rows`` token rows of either weight form (rows past one launch reuse it)."""
    return int(_lib.lib().oxr_lm_head_workspace_bytes(min(rows, MAX_ROWS_PACKED), vocab))


def lm_head_argmax(
    hidden: torch.Tensor, weight: Weight, *, return_logits: bool = False, predicted: torch.Tensor | None = None,
    logits: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """hidden bf16 ``[n, hidden]``, weight bf16 ``[vocab, hidden]`` (row-major or a
    :class:`~.gemm.PackedWeight`) -> (int64 ``[n]`` greedy ids, bf16 ``[n, vocab]`` logits when
    ``return_logits`` else None)."""
    packed = isinstance(weight, PackedWeight)
    wt = weight.data if packed else weight
    device = _lib.require_gpu(hidden, wt, name="lm_head_argmax")
    _lib.require(hidden.dtype == torch.bfloat16 and wt.dtype == torch.bfloat16, "bf16 operands required")
    _lib.require(hidden.dim() == 2 and len(weight.shape) == 2 and hidden.shape[1] == weight.shape[1], "shape mismatch")
    _lib.require(hidden.stride(1) == 1 and wt.is_contiguous(), "rows must be contiguous")
    n, k = hidden.shape
    vocab = weight.shape[0]
    if predicted is None:
        predicted = torch.empty(n, dtype=torch.int64, device=device)
    if return_logits and logits is None:
        logits = torch.empty(n, vocab, dtype=torch.bfloat16, device=device)
    need = workspace_bytes(n, vocab)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
    step = MAX_ROWS_PACKED if packed else MAX_ROWS
    for start in range(0, n, step):
        rows = min(step, n - start)
        _lib.call(
            "oxr_lm_head_argmax_packed" if packed else "oxr_lm_head_argmax", hidden[start:].data_ptr(), rows,
            wt.data_ptr(), k, vocab,
            logits[start:].data_ptr() if logits is not None else None, predicted[start:].data_ptr(),
            workspace.data_ptr(), workspace.numel(), _lib.stream(device),
        )
    return predicted, logits


def logits(hidden: torch.Tensor, weight: Weight) -> torch.Tensor:
    """``LanguageModel.logits``: bf16 ``hidden @ weight.T`` (language.py:213-214)."""
    return lm_head_argmax(hidden, weight, return_logits=True)[1]


def argmax(logits: torch.Tensor, *, out: torch.Tensor | None = None,
           workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``logits.argmax(dim=-1)`` (engine.py:726) for fp32 or bf16 logits ``[..., vocab]`` already in
    memory: int64 ``[...]``, the first index of each row's largest value (NaN counts as largest)."""
    device = _lib.require_gpu(logits, name="argmax")
    _lib.require(logits.dtype in (torch.float32, torch.bfloat16), "argmax: fp32 or bf16 logits")
    _lib.require(logits.dim() >= 1 and logits.shape[-1] > 0 and logits.stride(-1) == 1, "argmax: contiguous rows")
    vocab = logits.shape[-1]
    rows2d = logits.reshape(-1, vocab)
    _lib.require(rows2d.dim() == 2 and rows2d.stride(-1) == 1, "argmax: rows must be evenly strided")
    rows = rows2d.shape[0]
    if out is None:
        out = torch.empty(logits.shape[:-1], dtype=torch.int64, device=device)
    _lib.require(out.dtype == torch.int64 and out.numel() == rows and out.is_contiguous(), "argmax: out int64 [...]")
    need = int(_lib.lib().oxr_argmax_workspace_bytes(rows, vocab))
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
    dtype = 0 if logits.dtype == torch.float32 else 1  # OXR_DTYPE_F32 / OXR_DTYPE_BF16
    _lib.call("oxr_argmax", rows2d.data_ptr(), dtype, rows, vocab, rows2d.stride(0), out.data_ptr(),
              workspace.data_ptr(), workspace.numel() * workspace.element_size(), _lib.stream(device))
    return out
