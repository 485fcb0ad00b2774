"""gfx950 weight-streaming GEMMs and the fused LM-head argmax vs the oracle.

Projections: every output within 1 bf16 ulp of the exactly rounded product (fp32
accumulation in another order can only move a value across one rounding boundary), at the
verify shapes (M = 32, K = 2048 / 6144, N = 4096 / 2048 / 12288) and ragged ones.  LM head:
config 4 (hidden [256, 2048] ~N(0,1), weight [151936, 2048] ~N(0, 0.02)): logits within
|err| <= 2e-2 + 1e-2 |ref|, argmax identical wherever the exact top-2 margin exceeds 2e-2,
and exact first-index tie-breaking on planted duplicate rows.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, pkg
from oracle import bf16, lm_head as oracle_lm_head

pytestmark = pytest.mark.gpu
gemm = pkg("gemm")
lm_head = pkg("lm_head")

ATOL, RTOL = 2e-2, 1e-2


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _rand(g, *shape, std=1.0):
    return (torch.randn(*shape, generator=g, device="cuda") * std).to(torch.bfloat16)


def _ulp_bf16(x: np.ndarray) -> np.ndarray:
    mag = np.maximum(np.abs(x), 2.0**-126)
    return 2.0 ** (np.floor(np.log2(mag)) - 7)


def _exact(x: torch.Tensor, w: torch.Tensor) -> np.ndarray:
    return bf16.to_f32(_bits(x)).astype(np.float64) @ bf16.to_f32(_bits(w)).astype(np.float64).T


def _order_slack(x: torch.Tensor, w: torch.Tensor) -> np.ndarray:
    """fp32 accumulation in a different order moves a sum by a few fp32 ulps of the partial sums:
    bounded here by 1e-5 * sum_k |x_k w_k| (which only matters where the result cancels)."""
    return 1e-5 * (np.abs(bf16.to_f32(_bits(x)).astype(np.float64)) @ np.abs(bf16.to_f32(_bits(w)).astype(np.float64)).T)


@pytest.mark.parametrize("m,k,n", [(32, 2048, 4096), (32, 2048, 2048), (32, 6144, 2048), (1, 2048, 4096),
                                   (7, 2048, 160), (64, 2048, 2048), (100, 256, 512), (17, 128, 40)])
def test_linear_within_one_ulp(m: int, k: int, n: int) -> None:
    g = torch.Generator(device="cuda").manual_seed(m * 7 + n)
    x, w = _rand(g, m, k), _rand(g, n, k, std=0.02)
    announce("linear", m, k, n)
    y = gemm.linear(x, w)
    torch.cuda.synchronize()
    exact = _exact(x, w)
    got = bf16.to_f32(_bits(y)).astype(np.float64)
    err = np.abs(got - exact)
    assert (err <= _ulp_bf16(exact) + _order_slack(x, w)).all()
    assert (err <= ATOL + RTOL * np.abs(exact)).all()
    assert np.mean(err <= 0.5 * _ulp_bf16(exact) * 1.001) > 0.99  # almost always the exactly rounded value


@pytest.mark.parametrize("m,n", [(32, 6144), (5, 96)])
def test_linear_silu_mul_rounding_points(m: int, n: int) -> None:
    g = torch.Generator(device="cuda").manual_seed(n)
    x, w = _rand(g, m, 2048), _rand(g, 2 * n, 2048, std=0.02)
    announce("silu_mul", m, n)
    y = gemm.linear_silu_mul(x, w)
    torch.cuda.synchronize()
    exact = _exact(x, w)
    gate = bf16.round_f32(exact[:, :n].astype(np.float32)).astype(np.float64)
    up = bf16.round_f32(exact[:, n:].astype(np.float32)).astype(np.float64)
    silu = bf16.round_f32((gate / (1.0 + np.exp(-gate))).astype(np.float32)).astype(np.float64)
    want = bf16.round_f32((silu * up).astype(np.float32)).astype(np.float64)
    got = bf16.to_f32(_bits(y)).astype(np.float64)
    # One-ulp slack for each of the two GEMM outputs crossing a rounding boundary.
    assert (np.abs(got - want) <= ATOL + RTOL * np.abs(want)).all()
    assert np.mean(got == want) > 0.97


def test_linear_add_residual() -> None:
    g = torch.Generator(device="cuda").manual_seed(5)
    x, w, r = _rand(g, 32, 6144), _rand(g, 2048, 6144, std=0.02), _rand(g, 32, 2048)
    r0 = _bits(r).copy()
    announce("add residual")
    gemm.linear_add_(r, x, w)
    torch.cuda.synchronize()
    exact = _exact(x, w)
    prod = bf16.round_f32(exact.astype(np.float32)).astype(np.float64)
    want = bf16.round_f32((prod + bf16.to_f32(r0)).astype(np.float32)).astype(np.float64)
    got = bf16.to_f32(_bits(r)).astype(np.float64)
    # the product may land one ulp away (order slack), and the sum then rounds once more
    assert (np.abs(got - want) <= _ulp_bf16(prod) + _ulp_bf16(want) + _order_slack(x, w)).all()
    assert np.mean(got == want) > 0.98


def test_lm_head_config4_logits_and_argmax() -> None:
    g = torch.Generator(device="cuda").manual_seed(40)
    hidden, weight = _rand(g, 256, 2048), _rand(g, 151_936, 2048, std=0.02)
    announce("lm head config4")
    pred, logits = lm_head.lm_head_argmax(hidden, weight, return_logits=True)
    torch.cuda.synchronize()
    exact = _exact(hidden, weight)
    got = bf16.to_f32(_bits(logits)).astype(np.float64)
    assert (np.abs(got - exact) <= ATOL + RTOL * np.abs(exact)).all()
    ref_bits = bf16.from_f32(exact.astype(np.float32))
    ref_ids = oracle_lm_head.argmax(ref_bits)
    margin = oracle_lm_head.top2_margin(exact)
    sure = margin > ATOL
    pred = pred.cpu().numpy()
    assert sure.mean() > 0.8
    assert np.array_equal(pred[sure], ref_ids[sure])
    # Where the kernel's own bf16 logits decide, its id is exactly their first argmax.
    assert np.array_equal(pred, oracle_lm_head.argmax(_bits(logits)))


def test_lm_head_ties_take_lowest_index() -> None:
    g = torch.Generator(device="cuda").manual_seed(41)
    vocab, k = 4096 + 32, 2048
    hidden, weight = _rand(g, 8, k), _rand(g, vocab, k, std=0.02)
    # Rows 3, 9 (same tile), 77 and 4100 (other tiles) copy hidden[0] scaled: a clear, tied max for row 0.
    top = (hidden[0].float() * 0.05).to(torch.bfloat16)
    for v in (4100, 77, 9, 3):
        weight[v] = top
    weight[5] = (hidden[1].float() * 0.05).to(torch.bfloat16)
    weight[4099] = weight[5]
    announce("lm head ties")
    pred, logits = lm_head.lm_head_argmax(hidden, weight, return_logits=True)
    torch.cuda.synchronize()
    assert int(pred[0]) == 3 and int(pred[1]) == 5
    assert np.array_equal(pred.cpu().numpy(), oracle_lm_head.argmax(_bits(logits)))


@pytest.mark.parametrize("k", [2048, 6144])
def test_partial_gemm_then_add_rms_norm(k: int) -> None:
    """o_proj / down_proj path: k-split fp32 partials summed by the following add + RMSNorm:
    residual' = bf16(bf16(x @ w.T) + residual), h = bf16(w_n * bf16(residual' * rsqrt(mean sq + eps)))."""
    g = torch.Generator(device="cuda").manual_seed(k)
    m, n = 32, 2048
    x, w, r = _rand(g, m, k), _rand(g, n, k, std=0.02), _rand(g, m, n)
    wn = (0.5 + torch.rand(n, generator=g, device="cuda")).to(torch.bfloat16)
    r0 = _bits(r).copy()
    splits = gemm.partial_splits(n, k)
    assert splits >= 2
    partials = torch.full((splits, m, n), float("nan"), device="cuda")
    h = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    announce("partial gemm + add norm", k, splits)
    assert gemm.linear_partial(x, w, partials) == splits
    gemm.add_partials_rms_norm(partials, splits, r, wn, 1e-6, h)
    torch.cuda.synchronize()
    exact = _exact(x, w)
    prod = bf16.round_f32(exact.astype(np.float32)).astype(np.float64)
    want_r = bf16.round_f32((prod + bf16.to_f32(r0)).astype(np.float32)).astype(np.float64)
    got_r = bf16.to_f32(_bits(r)).astype(np.float64)
    assert (np.abs(got_r - want_r) <= _ulp_bf16(prod) + _ulp_bf16(want_r) + _order_slack(x, w)).all()
    assert np.mean(got_r == want_r) > 0.98
    # The norm of the residual actually stored (exact inputs): within the bf16 tolerance.
    rr = got_r.astype(np.float32)
    inv = (1.0 / np.sqrt((rr.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6))
    want_h = bf16.to_f32(_bits(wn)).astype(np.float64) * bf16.round_f32((rr * inv).astype(np.float32))
    got_h = bf16.to_f32(_bits(h)).astype(np.float64)
    assert (np.abs(got_h - want_h) <= ATOL + RTOL * np.abs(want_h)).all()
