"""Weight-streaming bf16 GEMMs with fused epilogues (csrc/gemm.hip) for the verify forward.

These replace the ``nn.Linear`` projections of the reference decoder layer (language.py:261,
268-269) and fold in the elementwise op that follows each projection there:

- ``linear``            ``x @ w.T``                       (qkv_proj, o_proj, down_proj)
- ``linear_silu_mul``   ``_silu_mul(x @ w.T)``            (gate_up_proj + SiLU*up, language.py:102-104)
- ``linear_add_``       ``residual += x @ w.T`` in bf16   (the add of ``_add_rms_norm``, language.py:94-99)
- ``linear_partial``    fp32 k-split partial sums of ``x @ w.T`` for weights too narrow to fill the chip
                        (o_proj, down_proj); ``add_partials_rms_norm`` finishes the sum, the residual add
                        and the next RMSNorm in one pass
"""

from __future__ import annotations

import torch

from . import _lib

EPI_STORE, EPI_SILU_MUL, EPI_ADD_RESIDUAL = 0, 1, 3
MAX_ROWS = 64  # token rows per launch; larger inputs are processed in slices


def _check(x: torch.Tensor, w: torch.Tensor, name: str) -> torch.device:
    device = _lib.require_gpu(x, w, name=name)
    _lib.require(x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16, f"{name}: bf16 operands required")
    _lib.require(x.dim() == 2 and w.dim() == 2 and x.shape[1] == w.shape[1], f"{name}: x [m, k] and w [n, k] required")
    _lib.require(x.stride(1) == 1 and w.is_contiguous(), f"{name}: rows must be contiguous")
    _lib.require(x.shape[1] % 128 == 0, f"{name}: k must be a multiple of 128")
    return device


def _run(x: torch.Tensor, w: torch.Tensor, n: int, epilogue: int, y: torch.Tensor, device: torch.device) -> None:
    m = x.shape[0]
    for start in range(0, m, MAX_ROWS):
        rows = min(MAX_ROWS, m - start)
        _lib.call("oxr_gemm_bf16", x[start:].data_ptr(), x.stride(0), rows, w.data_ptr(), w.shape[1], n, epilogue,
                  y[start:].data_ptr(), y.stride(0), _lib.stream(device))


def linear(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``x @ w.T`` in bf16 with fp32 accumulation (``F.linear`` without bias)."""
    device = _check(x, w, "linear")
    n = w.shape[0]
    if out is None:
        out = torch.empty(x.shape[0], n, dtype=torch.bfloat16, device=device)
    _lib.require(out.shape == (x.shape[0], n) and out.stride(1) == 1, "linear: out must be [m, n] with contiguous rows")
    _run(x, w, n, EPI_STORE, out, device)
    return out


def linear_silu_mul(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(g) * u`` where ``[g | u] = x @ w.T`` (``w`` is the fused gate_up weight, gate rows first)."""
    device = _check(x, w, "linear_silu_mul")
    _lib.require(w.shape[0] % 2 == 0, "linear_silu_mul: w must hold gate and up rows")
    n = w.shape[0] // 2
    if out is None:
        out = torch.empty(x.shape[0], n, dtype=torch.bfloat16, device=device)
    _lib.require(out.shape == (x.shape[0], n) and out.stride(1) == 1, "linear_silu_mul: out must be [m, n]")
    _run(x, w, n, EPI_SILU_MUL, out, device)
    return out


def linear_add_(residual: torch.Tensor, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``residual = bf16(bf16(x @ w.T) + residual)``, in place; returns ``residual``."""
    device = _check(x, w, "linear_add_")
    n = w.shape[0]
    _lib.require(residual.shape == (x.shape[0], n) and residual.dtype == torch.bfloat16 and residual.stride(1) == 1,
                 "linear_add_: residual must be bf16 [m, n]")
    _run(x, w, n, EPI_ADD_RESIDUAL, residual, device)
    return residual


def partial_splits(n: int, k: int) -> int:
    """How many k slices ``linear_partial`` uses for an ``[n, k]`` weight."""
    return int(_lib.lib().oxr_gemm_bf16_partial_splits(n, k))


def linear_partial(x: torch.Tensor, w: torch.Tensor, partials: torch.Tensor) -> int:
    """fp32 partial sums of ``x @ w.T`` over ``partial_splits(n, k)`` k slices into
    ``partials[:splits, :m, :n]``; returns the number of slices."""
    device = _check(x, w, "linear_partial")
    m, (n, k) = x.shape[0], w.shape
    _lib.require(m <= MAX_ROWS, "linear_partial: at most 64 rows")
    splits = partial_splits(n, k)
    _lib.require(partials.dtype == torch.float32 and partials.is_contiguous() and partials.numel() >= splits * m * n,
                 "linear_partial: partials must be contiguous fp32 with room for splits * m * n")
    _lib.call("oxr_gemm_bf16_partial", x.data_ptr(), x.stride(0), m, w.data_ptr(), k, n, partials.data_ptr(), splits,
              _lib.stream(device))
    return splits


def add_partials_rms_norm(partials: torch.Tensor, splits: int, residual: torch.Tensor, weight: torch.Tensor,
                          eps: float, out: torch.Tensor) -> torch.Tensor:
    """``residual = bf16(bf16(sum of partials) + residual)``; ``out = rms_norm(residual) * weight``
    (``_add_rms_norm``, language.py:94-99, taking a ``linear_partial`` result)."""
    device = _lib.require_gpu(partials, residual, weight, out, name="add_partials_rms_norm")
    rows, hidden = residual.shape
    _lib.call("oxr_add_partials_rms_norm", partials.data_ptr(), splits, rows, hidden, residual.data_ptr(),
              weight.data_ptr(), float(eps), out.data_ptr(), _lib.stream(device))
    return out
