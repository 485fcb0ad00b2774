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
it) or as a :class:`PackedMatrix` made once by :func:`pack_weight`, which the kernels stream
markedly faster; the results are bit-identical.  With a packed weight the token rows ``x`` and the
output may be packed too (the verify forward keeps them so between its kernels).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib


@dataclass(frozen=True)
class PackedMatrix:
    """A bf16 ``[rows, cols]`` matrix in the order the GEMM kernels stream their operands
    (csrc/gemm.hip): per 16-row tile and 128-column step, four contiguous 1 KiB blocks of MFMA
    fragments, so every load instruction reads contiguous memory.  Weights are packed once by
    :func:`pack_weight`; token rows travel between the verify forward's kernels in this layout
    (:func:`packed_rows` allocates them).  ``data`` is 1-D (the last tile padded) so it cannot be
    mistaken for a row-major matrix; it may hold more rows than ``rows`` (a buffer for up to N
    rows holds every smaller row count as a prefix)."""

    data: torch.Tensor
    rows: int
    cols: int

    @property
    def shape(self) -> tuple[int, int]:
        return (self.rows, self.cols)

    @property
    def device(self) -> torch.device:
        return self.data.device

    @property
    def dtype(self) -> torch.dtype:
        return self.data.dtype

    def to(self, device) -> "PackedMatrix":
        return PackedMatrix(self.data.to(device), self.rows, self.cols)

    def view_rows(self, rows: int) -> "PackedMatrix":
        """The first ``rows`` rows (same storage)."""
        _lib.require(-(-rows // 16) * 16 * self.cols <= self.data.numel(), "PackedMatrix.view_rows: beyond the buffer")
        return PackedMatrix(self.data, rows, self.cols)

    def unpack(self) -> torch.Tensor:
        """The row-major ``[rows, cols]`` matrix again (a view permutation; any device)."""
        tiles = -(-self.rows // 16)
        v = self.data[: tiles * 16 * self.cols].view(tiles, self.cols // 128, 4, 4, 16, 8)  # [tile, step, block, g, r, 8]
        return v.permute(0, 4, 1, 2, 3, 5).reshape(tiles * 16, self.cols)[: self.rows].contiguous()


PackedWeight = PackedMatrix  # a packed weight: rows = output features, cols = k
Weight = torch.Tensor | PackedMatrix
Rows = torch.Tensor | PackedMatrix


def packed_rows(rows: int, cols: int, device) -> PackedMatrix:
    """A zero-filled packed ``[rows, cols]`` bf16 buffer (cols a multiple of 128)."""
    _lib.require(cols % 128 == 0, "packed_rows: cols must be a multiple of 128")
    return PackedMatrix(torch.zeros(-(-rows // 16) * 16 * cols, dtype=torch.bfloat16, device=device), rows, cols)


def pack_weight(w: torch.Tensor) -> PackedMatrix:
    """Re-order a row-major bf16 ``[rows, k]`` weight (k a multiple of 128) on its GPU."""
    device = _lib.require_gpu(w, name="pack_weight")
    _lib.require(w.dtype == torch.bfloat16 and w.dim() == 2 and w.is_contiguous(), "pack_weight: contiguous bf16 [rows, k]")
    rows, k = w.shape
    _lib.require(k % 128 == 0, "pack_weight: k must be a multiple of 128")
    data = torch.empty(int(_lib.lib().oxr_packed_weight_elems(rows, k)), dtype=torch.bfloat16, device=device)
    _lib.call("oxr_pack_weight_bf16", w.data_ptr(), rows, k, data.data_ptr(), _lib.stream(device))
    return PackedMatrix(data, rows, k)


EPI_STORE, EPI_SILU_MUL, EPI_ADD_RESIDUAL = 0, 1, 3
X_PACKED, Y_PACKED = 1, 2  # OXR_GEMM_X_PACKED, OXR_GEMM_Y_PACKED
MAX_ROWS = 256  # token rows per call (the kernels take 64 per launch over the same weight); more are sliced


def _tensor(a: Weight) -> torch.Tensor:
    return a.data if isinstance(a, PackedMatrix) else a


def _check(x: Rows, w: Weight, name: str) -> torch.device:
    xt, wt = _tensor(x), _tensor(w)
    device = _lib.require_gpu(xt, wt, name=name)
    _lib.require(xt.dtype == torch.bfloat16 and wt.dtype == torch.bfloat16, f"{name}: bf16 operands required")
    _lib.require(len(x.shape) == 2 and len(w.shape) == 2 and x.shape[1] == w.shape[1],
                 f"{name}: x [m, k] and w [n, k] required")
    _lib.require(xt.stride(-1) == 1 and wt.is_contiguous(), f"{name}: rows must be contiguous")
    _lib.require(x.shape[1] % 128 == 0, f"{name}: k must be a multiple of 128")
    _lib.require(not isinstance(x, PackedMatrix) or isinstance(w, PackedMatrix), f"{name}: packed x needs a packed w")
    return device


def _run(x: Rows, w: Weight, n: int, epilogue: int, y: Rows, device: torch.device) -> None:
    m = x.shape[0]
    if isinstance(w, PackedMatrix):
        flags = (X_PACKED if isinstance(x, PackedMatrix) else 0) | (Y_PACKED if isinstance(y, PackedMatrix) else 0)
        if flags:
            _lib.require(m <= MAX_ROWS, f"packed rows: at most {MAX_ROWS} per call")
        ldx = 0 if isinstance(x, PackedMatrix) else x.stride(0)
        ldy = 0 if isinstance(y, PackedMatrix) else y.stride(0)
        for start in range(0, m, MAX_ROWS):
            rows = min(MAX_ROWS, m - start)
            xp = x.data.data_ptr() if isinstance(x, PackedMatrix) else x[start:].data_ptr()
            yp = y.data.data_ptr() if isinstance(y, PackedMatrix) else y[start:].data_ptr()
            _lib.call("oxr_gemm_bf16_packed", xp, ldx, rows, w.data.data_ptr(), w.shape[1], n, epilogue, yp, ldy,
                      flags, _lib.stream(device))
        return
    _lib.require(not isinstance(y, PackedMatrix), "packed output needs a packed w")
    for start in range(0, m, MAX_ROWS):
        rows = min(MAX_ROWS, m - start)
        _lib.call("oxr_gemm_bf16", x[start:].data_ptr(), x.stride(0), rows, w.data_ptr(), w.shape[1], n, epilogue,
                  y[start:].data_ptr(), y.stride(0), _lib.stream(device))


def _check_out(out: Rows, m: int, n: int, name: str) -> None:
    if isinstance(out, PackedMatrix):
        _lib.require(out.shape == (m, n) and out.data.numel() >= -(-m // 16) * 16 * n, f"{name}: packed out too small")
    else:
        _lib.require(out.shape == (m, n) and out.stride(1) == 1, f"{name}: out must be [m, n] with contiguous rows")


def linear(x: Rows, w: Weight, out: Rows | None = None) -> Rows:
    """``x @ w.T`` in bf16 with fp32 accumulation (``F.linear`` without bias)."""
    device = _check(x, w, "linear")
    n = w.shape[0]
    if out is None:
        out = torch.empty(x.shape[0], n, dtype=torch.bfloat16, device=device)
    _check_out(out, x.shape[0], n, "linear")
    _run(x, w, n, EPI_STORE, out, device)
    return out


def linear_silu_mul(x: Rows, w: Weight, out: Rows | None = None) -> Rows:
    """``silu(g) * u`` where ``[g | u] = x @ w.T`` (``w`` is the fused gate_up weight, gate rows first)."""
    device = _check(x, w, "linear_silu_mul")
    _lib.require(w.shape[0] % 2 == 0, "linear_silu_mul: w must hold gate and up rows")
    n = w.shape[0] // 2
    if out is None:
        out = torch.empty(x.shape[0], n, dtype=torch.bfloat16, device=device)
    _check_out(out, x.shape[0], n, "linear_silu_mul")
    _run(x, w, n, EPI_SILU_MUL, out, device)
    return out


def linear_add_(residual: torch.Tensor, x: Rows, w: Weight) -> torch.Tensor:
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


def linear_partial(x: Rows, w: Weight, partials: torch.Tensor) -> int:
    """fp32 partial sums of ``x @ w.T`` over ``partial_splits(n, k)`` k slices into
    ``partials[:splits, :m, :n]``; returns the number of slices."""
    device = _check(x, w, "linear_partial")
    m, (n, k) = x.shape[0], w.shape
    _lib.require(m <= MAX_ROWS, f"linear_partial: at most {MAX_ROWS} rows")
    splits = partial_splits(n, k)
    _lib.require(partials.dtype == torch.float32 and partials.is_contiguous() and partials.numel() >= splits * m * n,
                 "linear_partial: partials must be contiguous fp32 with room for splits * m * n")
    if isinstance(w, PackedMatrix):
        xp = isinstance(x, PackedMatrix)
        _lib.call("oxr_gemm_bf16_partial_packed", _tensor(x).data_ptr(), 0 if xp else x.stride(0), m,
                  w.data.data_ptr(), k, n, partials.data_ptr(), splits, X_PACKED if xp else 0, _lib.stream(device))
    else:
        _lib.call("oxr_gemm_bf16_partial", x.data_ptr(), x.stride(0), m, w.data_ptr(), k, n, partials.data_ptr(),
                  splits, _lib.stream(device))
    return splits


def add_partials_rms_norm(partials: torch.Tensor, splits: int, residual: torch.Tensor, weight: torch.Tensor,
                          eps: float, out: Rows, *, residual_in: torch.Tensor | None = None) -> Rows:
    """``residual = bf16(bf16(sum of partials) + residual)``; ``out = rms_norm(residual) * weight``
    (``_add_rms_norm``, language.py:94-99, taking a ``linear_partial`` result).  ``out`` may be a
    :class:`PackedMatrix` (the next GEMM's packed x).  With ``residual_in`` the residual is read from
    there and the sum stored to ``residual`` (after ``mlp.mlp_block``)."""
    device = _lib.require_gpu(partials, residual, weight, _tensor(out), name="add_partials_rms_norm")
    rows, hidden = residual.shape
    _check_out(out, rows, hidden, "add_partials_rms_norm")
    packed = 1 if isinstance(out, PackedMatrix) else 0
    if residual_in is None:
        _lib.call("oxr_add_partials_rms_norm", partials.data_ptr(), splits, rows, hidden, residual.data_ptr(),
                  weight.data_ptr(), float(eps), _tensor(out).data_ptr(), packed, _lib.stream(device))
    else:
        _lib.require(tuple(residual_in.shape) == (rows, hidden) and residual_in.is_contiguous()
                     and residual_in.dtype == torch.bfloat16, "add_partials_rms_norm: residual_in like residual")
        _lib.call("oxr_add_partials_rms_norm_from", partials.data_ptr(), splits, rows, hidden,
                  residual_in.data_ptr(), residual.data_ptr(), weight.data_ptr(), float(eps),
                  _tensor(out).data_ptr(), packed, _lib.stream(device))
    return out
