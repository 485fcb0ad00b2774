"""The MFMA 16x16x32 bf16 operand/result lane layout the attention and GEMM kernels assume."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, pkg

pytestmark = pytest.mark.gpu
_lib = pkg("_lib")


def test_mfma_16x16x32_bf16_layout() -> None:
    rng = np.random.default_rng(0)
    a = torch.from_numpy(rng.integers(-4, 5, size=(16, 32)).astype(np.float32)).to(torch.bfloat16).cuda()
    b = torch.from_numpy(rng.integers(-4, 5, size=(32, 16)).astype(np.float32)).to(torch.bfloat16).cuda()
    c = torch.zeros(16, 16, dtype=torch.float32, device="cuda")
    announce("mfma layout")
    _lib.call("oxr_selftest_mfma_layout", a.data_ptr(), b.data_ptr(), c.data_ptr(), _lib.stream(c.device))
    torch.cuda.synchronize()
    want = a.float().cpu() @ b.float().cpu()  # small integers: exact in fp32
    assert torch.equal(c.cpu(), want)
