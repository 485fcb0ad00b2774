"""The drop-in boundary refuses CPU tensors instead of falling back to a CPU path
(the reference dispatches CPU tensors to torch code, kernels.py:111-112; this build
has none), and validates shapes on the host before any launch."""

from __future__ import annotations

import pytest
import torch

from conftest import pkg

kernels = pkg("kernels")
spec = pkg("speculative")


def _bf(*shape):
    return torch.zeros(*shape, dtype=torch.bfloat16)


def test_qk_norm_rope_store_rejects_cpu_tensors() -> None:
    w = _bf(128)
    with pytest.raises(RuntimeError, match="GPU"):
        kernels.qk_norm_rope_store(_bf(1, 4 * 128), w, w, _bf(1, 64), _bf(1, 64), 1e-6, _bf(1, 1, 1, 128),
                                   _bf(1, 1, 1, 128), torch.zeros(1, dtype=torch.long), 2, 1, 128, need_kv=False)


def test_speculative_rejects_cpu_tensors() -> None:
    h = torch.zeros(2, 8, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        spec.propose_batch(h, torch.zeros(2, dtype=torch.int32), 3)
