"""Pins the LM-head / argmax oracle (oracle/lm_head.py).

- One-hot hidden rows read single weight columns back exactly (orientation: logits[i, v]
  = sum_k hidden[i, k] * weight[v, k], not the transpose).
- Ties go to the first index; NaN wins (torch.argmax's convention) -- checked against torch.
- The top-2 margin is the difference of the two largest values.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import bf16, lm_head


def test_one_hot_rows_pick_weight_columns() -> None:
    rng = np.random.default_rng(0)
    w = bf16.from_f32(rng.standard_normal((50, 16)).astype(np.float32))
    hidden = np.zeros((3, 16), dtype=np.float32)
    hidden[0, 2] = hidden[1, 7] = hidden[2, 15] = 1.0
    out = lm_head.logits(bf16.from_f32(hidden), w)
    assert np.array_equal(out, w[:, [2, 7, 15]].T)


def test_argmax_first_index_and_nan_like_torch() -> None:
    rows = np.array([[1.0, 3.0, 3.0, 2.0], [0.0, -0.0, -1.0, -0.0], [1.0, np.nan, 5.0, np.nan], [-2.0, -2.0, -2.0, -3.0]],
                    dtype=np.float32)
    bits = bf16.from_f32(rows)
    want = torch.from_numpy(bf16.to_f32(bits)).to(torch.bfloat16).argmax(-1).numpy()
    assert lm_head.argmax(bits).tolist() == want.tolist() == [1, 0, 1, 0]


def test_top2_margin() -> None:
    v = np.array([[0.5, 2.0, 1.25], [3.0, 3.0, 0.0]])
    assert lm_head.top2_margin(v).tolist() == [0.75, 0.0]
