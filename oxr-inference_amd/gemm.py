"""Weight-streaming bf16 GEMMs with fused epilogues (csrc/gemm.hip) for the verify forward.

These replace the ``nn.Linear`` projections of the reference decoder layer (language.py:261,
268-269) and fold in the elementwise op that follows each projection there:

- ``linear``            ``x @ w.T``                       (qkv_proj, o_proj, down_proj)
- ``linear_silu_mul``   ``_silu_mul(x @ w.T)``            (gate_up_proj + SiLU*up, language.py:102-104)
- ``linear_add_``       ``residual += x @ w.T`` in bf16   (the add of ``_add_rms_norm``, language.py:94-99)
- ``linear_partial``    fp32 k-split partial sums of ``x @ w.T`` for weights too narrow to fill the chip
                        (o_proj, down_proj); ``add_partials_rms_norm`` finishes the sum, the residual add
                        and the next RMSNorm in one pass

Every function takes the weight either row-major (a ``torch.Tensor`` ``[n, k]``, as nn.Linear holds
it) or as a :class:`PackedWeight` made once by :func:`pack_weight`, which the kernels stream
markedly faster; the results are bit-identical.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib


@dataclass(frozen=True)
class PackedWeight:
    """A bf16 ``[rows, k]`` weight re-ordered once into the order the GEMM kernels stream it
    (``oxr_pack_weight_bf16``): per 16-row tile and 128-column step, four contiguous 1 KiB blocks
    of MFMA fragments, so every load instruction reads contiguous memory.  ``data`` is 1-D (the
    last tile zero-padded) so it cannot be mistaken for a row-major matrix."""

    data: torch.Tensor
    rows: int
    k: int

    @property
    def shape(self) -> tuple[int, int]:
        return (self.rows, self.k)

    @property
    def device(self) -> torch.device:
        return self.data.device

    @property
    def dtype(self) -> torch.dtype:
        return self.data.dtype

    def to(self, device) -> "PackedWeight":
        return PackedWeight(self.data.to(device), self.rows, self.k)

    def unpack(self) -> torch.Tensor:
        """The row-major ``[rows, k]`` weight again (a view permutation; any device)."""
        tiles = -(-self.rows // 16)
        v = self.data.view(tiles, self.k // 128, 4, 4, 16, 8)  # [tile, step, block, g, r, 8]
        return v.permute(0, 4, 1, 2, 3, 5).reshape(tiles * 16, self.k)[: self.rows].contiguous()


Weight = torch.Tensor | PackedWeight


def pack_weight(w: torch.Tensor) -> PackedWeight:
    """Re-order a row-major bf16 ``[rows, k]`` weight (k a multiple of 128) on its GPU."""
    device = _lib.require_gpu(w, name="pack_weight")
    _lib.require(w.dtype == torch.bfloat16 and w.dim() == 2 and w.is_contiguous(), "pack_weight: contiguous bf16 [rows, k]")
    rows, k = w.shape
    _lib.require(k % 128 == 0, "pack_weight: k must be a multiple of 128")
    data = torch.empty(int(_lib.lib().oxr_packed_weight_elems(rows, k)), dtype=torch.bfloat16, device=device)
    _lib.call("oxr_pack_weight_bf16", w.data_ptr(), rows, k, data.data_ptr(), _lib.stream(device))
    return PackedWeight(data, rows, k)

EPI_STORE, EPI_SILU_MUL, EPI_ADD_RESIDUAL = 0, 1, 3
MAX_ROWS = 64  # token rows per launch; larger inputs are processed in slices


def _check(x: torch.Tensor, w: Weight, name: str) -> torch.device:
    wt = w.data if isinstance(w, PackedWeight) else w
    device = _lib.require_gpu(x, wt, name=name)
    _lib.require(x.dtype == torch.bfloat16 and wt.dtype == torch.bfloat16, f"{name}: bf16 operands required")
    _lib.require(x.dim() == 2 and len(w.shape) == 2 and x.shape[1] == w.shape[1], f"{name}: x [m, k] and w [n, k] required")
    _lib.require(x.stride(1) == 1 and wt.is_contiguous(), f"{name}: rows must be contiguous")
    _lib.require(x.shape[1] % 128 == 0, f"{name}: k must be a multiple of 128")
    return device


def _entry(name: str, w: Weight) -> str:
    return name + "_packed" if isinstance(w, PackedWeight) else name


def _ptr(w: Weight) -> int:
    return w.data.data_ptr() if isinstance(w, PackedWeight) else w.data_ptr()


def _run(x: torch.Tensor, w: Weight, n: int, epilogue: int, y: torch.Tensor, device: torch.device) -> None:
    m = x.shape[0]
    for start in range(0, m, MAX_ROWS):
        rows = min(MAX_ROWS, m - start)
        _lib.call(_entry("oxr_gemm_bf16", w), x[start:].data_ptr(), x.stride(0), rows, _ptr(w), w.shape[1], n,
                  epilogue, y[start:].data_ptr(), y.stride(0), _lib.stream(device))


def linear(x: torch.Tensor, w: Weight, out: torch.Tensor | None = None) -> torch.Tensor:
    """``x @ w.T`` in bf16 with fp32 accumulation (``F.linear`` without bias)."""
    device = _check(x, w, "linear")
    n = w.shape[0]
    if out is None:
        out = torch.empty(x.shape[0], n, dtype=torch.bfloat16, device=device)
    _lib.require(out.shape == (x.shape[0], n) and out.stride(1) == 1, "linear: out must be [m, n] with contiguous rows")
    _run(x, w, n, EPI_STORE, out, device)
    return out


def linear_silu_mul(x: torch.Tensor, w: Weight, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(g) * u`` where ``[g | u] = x @ w.T`` (``w`` is the fused gate_up weight, gate rows first)."""
    device = _check(x, w, "linear_silu_mul")
    _lib.require(w.shape[0] % 2 == 0, "linear_silu_mul: w must hold gate and up rows")
    n = w.shape[0] // 2
    if out is None:
        out = torch.empty(x.shape[0], n, dtype=torch.bfloat16, device=device)
    _lib.require(out.shape == (x.shape[0], n) and out.stride(1) == 1, "linear_silu_mul: out must be [m, n]")
    _run(x, w, n, EPI_SILU_MUL, out, device)
    return out


def linear_add_(residual: torch.Tensor, x: torch.Tensor, w: Weight) -> torch.Tensor:
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


def linear_partial(x: torch.Tensor, w: Weight, partials: torch.Tensor) -> int:
    """fp32 partial sums of ``x @ w.T`` over ``partial_splits(n, k)`` k slices into
    ``partials[:splits, :m, :n]``; returns the number of slices."""
    device = _check(x, w, "linear_partial")
    m, (n, k) = x.shape[0], w.shape
    _lib.require(m <= MAX_ROWS, "linear_partial: at most 64 rows")
    splits = partial_splits(n, k)
    _lib.require(partials.dtype == torch.float32 and partials.is_contiguous() and partials.numel() >= splits * m * n,
                 "linear_partial: partials must be contiguous fp32 with room for splits * m * n")
    _lib.call(_entry("oxr_gemm_bf16_partial", w), x.data_ptr(), x.stride(0), m, _ptr(w), k, n, partials.data_ptr(),
              splits, _lib.stream(device))
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
