"""A decoder layer's MLP block in one launch (csrc/mlp_block.hip) for the verify step's token rows.

``DecoderLayer._mlp`` (oxr_runtime/language.py:266-269): the post-attention ``_add_rms_norm`` of
the o_proj output (94-99), ``gate_up_proj``, ``_silu_mul`` (102-104) and ``down_proj``, for up to 32
token rows of the config-5 decoder (hidden 2048, intermediate 6144) on an MI355X.  The three-launch
form (``gemm.add_partials_rms_norm``, ``gemm.linear_silu_mul``, ``gemm.linear_partial``) serves every
other shape.  Each XCD of the chip owns an eighth of the intermediate dimension, so the block runs
as one launch with its hand-offs inside each XCD; its output is 8 fp32 partial slices that the next
norm sums, and the new residual goes to a second buffer (``residual_out``).

The gate_up weight is used with its rows interleaved by 8 (:func:`interleave_gate_up`): each 16-row
tile then holds the gate and up rows of the same 8 intermediate columns, so a workgroup applies
``silu(gate) * up`` to the columns it computed.
"""

from __future__ import annotations

import torch

from . import _lib
from .gemm import PackedMatrix

MAX_ROWS = 32
SPLITS_OUT = 8   # partial slices of the block's output
ERROR_WORD = 512  # uint32 index of the workspace's error word


def interleave_gate_up(gate_up: torch.Tensor) -> torch.Tensor:
    """The fused gate_up weight ``[2 I, H]`` (gate rows, then up rows; language.py:238) with its rows
    interleaved by 8: row ``16 j + i`` is gate row ``8 j + i`` for ``i < 8``, up row ``8 j + i - 8``
    otherwise."""
    two_i, hidden = gate_up.shape
    _lib.require(two_i % 16 == 0, "interleave_gate_up: 2 * intermediate must be a multiple of 16")
    return gate_up.view(2, two_i // 16, 8, hidden).transpose(0, 1).reshape(two_i, hidden).contiguous()


def supported(rows: int, hidden: int, intermediate: int, o_splits: int = 4) -> bool:
    """Whether :func:`mlp_block` takes this shape on the current device."""
    return bool(_lib.lib().oxr_mlp_block_supported(rows, hidden, intermediate, o_splits))


def workspace(device) -> torch.Tensor:
    """A zeroed workspace; one serves every later call on its stream."""
    return torch.zeros(int(_lib.lib().oxr_mlp_block_workspace_bytes()), dtype=torch.uint8, device=device)


def error_bits(ws: torch.Tensor) -> int:
    """The workspace's error word (0: every launch so far met its placement and waits); synchronises."""
    return int(ws[4 * ERROR_WORD: 4 * ERROR_WORD + 4].view(torch.int32).item())


def mlp_block(o_partials: torch.Tensor, o_splits: int, residual_in: torch.Tensor, post_norm: torch.Tensor, eps: float,
              gate_up_interleaved: PackedMatrix, down: PackedMatrix, residual_out: torch.Tensor,
              partials_out: torch.Tensor, ws: torch.Tensor) -> torch.Tensor:
    """``residual_out = bf16(bf16(sum of o_partials) + residual_in)``, then the MLP of
    ``rms_norm(residual_out) * post_norm`` into ``partials_out`` (fp32 ``[8, rows, hidden]``);
    returns ``partials_out``."""
    device = _lib.require_gpu(o_partials, residual_in, post_norm, gate_up_interleaved.data, down.data, residual_out,
                              partials_out, ws, name="mlp_block")
    rows, hidden = residual_in.shape
    intermediate = down.cols
    _lib.require(isinstance(gate_up_interleaved, PackedMatrix) and isinstance(down, PackedMatrix),
                 "mlp_block: packed weights required")
    _lib.require(gate_up_interleaved.shape == (2 * intermediate, hidden) and down.shape == (hidden, intermediate),
                 "mlp_block: weight shapes")
    _lib.require(residual_in.is_contiguous() and residual_out.is_contiguous()
                 and tuple(residual_out.shape) == (rows, hidden), "mlp_block: contiguous [rows, hidden] residuals")
    _lib.require(o_partials.dtype == torch.float32 and o_partials.is_contiguous()
                 and o_partials.numel() >= o_splits * rows * hidden, "mlp_block: o_partials fp32 [o_splits, rows, hidden]")
    _lib.require(partials_out.dtype == torch.float32 and partials_out.is_contiguous()
                 and partials_out.numel() >= SPLITS_OUT * rows * hidden, "mlp_block: partials_out fp32 [8, rows, hidden]")
    _lib.call("oxr_mlp_block", o_partials.data_ptr(), o_splits, residual_in.data_ptr(), rows, hidden, intermediate,
              post_norm.data_ptr(), float(eps), gate_up_interleaved.data.data_ptr(), down.data.data_ptr(),
              residual_out.data_ptr(), partials_out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream(device))
    return partials_out
