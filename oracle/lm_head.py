"""LM head, greedy argmax and acceptance on the CPU (test infrastructure only).

- ``logits``: language.py:213-214, ``lm_head(hidden)`` -- a bf16 ``nn.Linear`` whose output is
  the fp32 dot product rounded to bf16.  Computed here in float64 then rounded.
- ``argmax``: decode_graph.py:167 / engine.py:726, ``argmax(dim=-1)`` over the bf16 logits:
  first index of the maximum.
- ``top2_margin``: the gap between the largest and second-largest logit of each row, the
  quantity the reference's scripts/divergence.py:70-75 reports at a divergence; ids are only
  required to match where it exceeds the logit tolerance.
"""

from __future__ import annotations

import numpy as np

from . import bf16


def logits_exact(hidden_bits: np.ndarray, weight_bits: np.ndarray) -> np.ndarray:
    """float64 [n, vocab] = hidden @ weight.T (bf16 inputs, no intermediate rounding)."""
    h = bf16.to_f32(hidden_bits).astype(np.float64)
    w = bf16.to_f32(weight_bits).astype(np.float64)
    return h @ w.T


def logits(hidden_bits: np.ndarray, weight_bits: np.ndarray) -> np.ndarray:
    """bf16 bits [n, vocab]: the exact product rounded once to bf16."""
    return bf16.from_f32(logits_exact(hidden_bits, weight_bits).astype(np.float32))


def argmax(logit_bits: np.ndarray) -> np.ndarray:
    """First index of the largest bf16 value per row (int64)."""
    return np.argmax(bf16.to_f32(logit_bits), axis=-1).astype(np.int64)


def top2_margin(values: np.ndarray) -> np.ndarray:
    part = np.partition(values, -2, axis=-1)
    return part[..., -1] - part[..., -2]
