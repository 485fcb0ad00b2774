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
_lib = pkg("_lib")

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
                                   (7, 2048, 160), (64, 2048, 2048), (100, 256, 512), (17, 128, 40),
                                   (72, 2048, 4096)])
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


@pytest.mark.parametrize("rows,k", [(4096, 2048), (40, 256), (1000, 128)])
def test_pack_weight_round_trip(rows: int, k: int) -> None:
    """The packed layout is a pure re-ordering (zero-padded last tile): unpacking gives the
    weight back bit for bit, and block i of (tile t, step q) holds w[16t + r][128q + 32i + 8g, +8)
    at lane 16g + r."""
    g = torch.Generator(device="cuda").manual_seed(rows)
    w = _rand(g, rows, k)
    announce("pack", rows, k)
    p = gemm.pack_weight(w)
    torch.cuda.synchronize()
    assert p.data.numel() == -(-rows // 16) * 16 * k
    assert torch.equal(p.unpack().view(torch.int16), w.view(torch.int16))
    flat = p.data.view(torch.int16).cpu().numpy()
    wb = w.view(torch.int16).cpu().numpy()
    t, q, i, lane = rows // 16 - 1, k // 128 - 1, 2, 37
    r, gg = lane % 16, lane // 16
    off = (((t * (k // 128) + q) * 4 + i) * 64 + lane) * 8
    assert np.array_equal(flat[off:off + 8], wb[16 * t + r, 128 * q + 32 * i + 8 * gg:][:8])
    tiles = -(-rows // 16)
    full = flat.reshape(tiles, k // 128, 4, 4, 16, 8).transpose(0, 4, 1, 2, 3, 5).reshape(tiles * 16, k)
    assert not full[rows:].any()  # the last tile's padding rows are zero


@pytest.mark.parametrize("m,k,n,epi", [(32, 2048, 4096, "store"), (32, 2048, 6144, "silu"), (32, 2048, 2048, "partial"),
                                       (32, 6144, 2048, "partial"), (32, 6144, 2048, "add"), (7, 256, 40, "store"),
                                       (64, 512, 96, "silu"), (17, 128, 40, "partial")])
def test_packed_weight_gemm_bit_identical(m: int, k: int, n: int, epi: str) -> None:
    """Packed and row-major weights run the same arithmetic in the same order."""
    g = torch.Generator(device="cuda").manual_seed(m + k + n)
    x = _rand(g, m, k)
    w = _rand(g, 2 * n if epi == "silu" else n, k, std=0.02)
    p = gemm.pack_weight(w)
    announce("packed gemm", m, k, n, epi)
    if epi == "partial":
        splits = gemm.partial_splits(n, k)
        a = torch.full((splits, m, n), float("nan"), device="cuda")
        b = torch.full((splits, m, n), float("nan"), device="cuda")
        gemm.linear_partial(x, w, a)
        gemm.linear_partial(x, p, b)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
        return
    if epi == "add":
        r = _rand(g, m, n)
        a, b = r.clone(), r.clone()
        gemm.linear_add_(a, x, w)
        gemm.linear_add_(b, x, p)
    else:
        fn = gemm.linear if epi == "store" else gemm.linear_silu_mul
        a, b = fn(x, w), fn(x, p)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("m,k,n,epi", [(32, 2048, 4096, "store"), (32, 2048, 6144, "silu"), (32, 2048, 2048, "partial"),
                                       (32, 6144, 2048, "partial"), (7, 256, 128, "store"), (20, 512, 256, "silu"),
                                       (17, 128, 40, "partial")])
def test_packed_rows_bit_identical(m: int, k: int, n: int, epi: str) -> None:
    """Token rows in the packed layout (x read packed, y written packed) give the row-major results
    bit for bit; rows past m in the last tile are padding and may hold anything."""
    g = torch.Generator(device="cuda").manual_seed(3 * m + k + n)
    x = _rand(g, m, k)
    w = gemm.pack_weight(_rand(g, 2 * n if epi == "silu" else n, k, std=0.02))
    xp = gemm.pack_weight(x)  # the same layout as packed token rows
    if m % 16:  # poison the last tile's padding rows: their results must never be stored
        tiles = -(-m // 16)
        xp.data.view(tiles, k // 128, 4, 4, 16, 8)[-1, :, :, :, m % 16:, :] = float("nan")
    announce("packed rows", m, k, n, epi)
    if epi == "partial":
        splits = gemm.partial_splits(n, k)
        a = torch.full((splits, m, n), float("nan"), device="cuda")
        b = torch.full((splits, m, n), float("nan"), device="cuda")
        gemm.linear_partial(x, w, a)
        gemm.linear_partial(xp, w, b)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
        return
    fn = gemm.linear if epi == "store" else gemm.linear_silu_mul
    a = fn(x, w)
    b = fn(xp, w, out=gemm.packed_rows(m, n, "cuda"))
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.unpack().view(torch.int16))


@pytest.mark.parametrize("rows,hidden", [(32, 2048), (12, 512), (40, 1024)])
def test_norms_packed_output(rows: int, hidden: int) -> None:
    """The three norm entry points write the same values packed as row-major."""
    g = torch.Generator(device="cuda").manual_seed(rows + hidden)
    lib = _lib
    st = lib.stream(torch.device("cuda"))
    x, wn = _rand(g, rows, hidden), (0.5 + torch.rand(hidden, generator=g, device="cuda")).to(torch.bfloat16)
    announce("norms packed", rows, hidden)
    a = torch.empty(rows, hidden, dtype=torch.bfloat16, device="cuda")
    b = gemm.packed_rows(rows, hidden, "cuda")
    lib.call("oxr_rms_norm", x.data_ptr(), hidden, rows, hidden, wn.data_ptr(), 1e-6, a.data_ptr(), hidden, 0, st)
    lib.call("oxr_rms_norm", x.data_ptr(), hidden, rows, hidden, wn.data_ptr(), 1e-6, b.data.data_ptr(), 0, 1, st)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.unpack().view(torch.int16))
    table = _rand(g, 100, hidden)
    ids = torch.randint(0, 100, (rows,), generator=g, device="cuda")
    ra, rb = torch.empty_like(a), torch.empty_like(a)
    lib.call("oxr_embed_rms_norm", ids.data_ptr(), rows, table.data_ptr(), 100, hidden, wn.data_ptr(), 1e-6,
             ra.data_ptr(), a.data_ptr(), 0, st)
    lib.call("oxr_embed_rms_norm", ids.data_ptr(), rows, table.data_ptr(), 100, hidden, wn.data_ptr(), 1e-6,
             rb.data_ptr(), b.data.data_ptr(), 1, st)
    torch.cuda.synchronize()
    assert torch.equal(ra, rb) and torch.equal(a.view(torch.int16), b.unpack().view(torch.int16))
    parts = torch.randn(4, rows, hidden, generator=g, device="cuda")
    r1, r2 = x.clone(), x.clone()
    gemm.add_partials_rms_norm(parts, 4, r1, wn, 1e-6, a)
    gemm.add_partials_rms_norm(parts, 4, r2, wn, 1e-6, b)
    torch.cuda.synchronize()
    assert torch.equal(r1, r2) and torch.equal(a.view(torch.int16), b.unpack().view(torch.int16))


@pytest.mark.parametrize("m,vocab,k", [(32, 151_936, 2048), (8, 4096 + 40, 2048), (40, 1000, 512), (3, 72, 384)])
def test_packed_lm_head_bit_identical(m: int, vocab: int, k: int) -> None:
    """Packed LM head (persistent kernel for m <= 32 and hidden 512/1024/2048, tile kernel otherwise):
    the same ids and bf16 logits as the row-major weight, including a vocab that is not a multiple
    of 16 (the padded rows of the last tile never win)."""
    g = torch.Generator(device="cuda").manual_seed(vocab)
    hidden, weight = _rand(g, m, k), _rand(g, vocab, k, std=0.02)
    weight[vocab - 1] = (hidden[0].float() * 0.05).to(torch.bfloat16)  # row 0's max in the last, partial tile
    p = gemm.pack_weight(weight)
    announce("packed lm head", m, vocab, k)
    ia, la = lm_head.lm_head_argmax(hidden, weight, return_logits=True)
    ib, lb = lm_head.lm_head_argmax(hidden, p, return_logits=True)
    torch.cuda.synchronize()
    assert int(ib[0]) == vocab - 1
    assert torch.equal(ia, ib)
    assert torch.equal(la.view(torch.int16), lb.view(torch.int16))


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


@pytest.mark.parametrize("rows", [256, 64, 40, 200])
def test_lm_head_wide_rows_packed(rows) -> None:
    """33..256 token rows with the packed weight: one launch reads the weight once (32x32x16
    MFMA, token rows staged in LDS).  Config 4 at 256 rows, and row counts that leave partial
    token tiles; logits within tolerance of the exact product, ids exact where the margin is clear
    and always the first argmax of the kernel's own bf16 logits."""
    g = torch.Generator(device="cuda").manual_seed(50 + rows)
    hidden, weight = _rand(g, rows, 2048), _rand(g, 151_936, 2048, std=0.02)
    packed = gemm.pack_weight(weight)
    announce("lm head wide", rows)
    pred, logits = lm_head.lm_head_argmax(hidden, packed, return_logits=True)
    pred_only, _ = lm_head.lm_head_argmax(hidden, packed)
    torch.cuda.synchronize()
    exact = _exact(hidden, weight)
    got = bf16.to_f32(_bits(logits)).astype(np.float64)
    assert (np.abs(got - exact) <= ATOL + RTOL * np.abs(exact)).all()
    ref_ids = oracle_lm_head.argmax(bf16.from_f32(exact.astype(np.float32)))
    sure = oracle_lm_head.top2_margin(exact) > ATOL
    pred = pred.cpu().numpy()
    assert sure.mean() > 0.8
    assert np.array_equal(pred[sure], ref_ids[sure])
    assert np.array_equal(pred, oracle_lm_head.argmax(_bits(logits)))
    assert np.array_equal(pred, pred_only.cpu().numpy())


@pytest.mark.parametrize("rows", [32, 8, 1])
def test_lm_head_step_rows_exact(rows) -> None:
    """The verify step's own LM head (persistent kernel, up to 32 token rows, packed weight) at the
    full vocab: logits within tolerance of the exact product, ids equal to the oracle's argmax of the
    exact logits where the margin is clear, and always the first argmax of the kernel's bf16 logits."""
    g = torch.Generator(device="cuda").manual_seed(70 + rows)
    hidden, weight = _rand(g, rows, 2048), _rand(g, 151_936, 2048, std=0.02)
    packed = gemm.pack_weight(weight)
    announce("lm head step rows", rows)
    pred, logits = lm_head.lm_head_argmax(hidden, packed, return_logits=True)
    torch.cuda.synchronize()
    exact = _exact(hidden, weight)
    got = bf16.to_f32(_bits(logits)).astype(np.float64)
    assert (np.abs(got - exact) <= ATOL + RTOL * np.abs(exact)).all()
    ref_ids = oracle_lm_head.argmax(bf16.from_f32(exact.astype(np.float32)))
    sure = oracle_lm_head.top2_margin(exact) > ATOL
    pred = pred.cpu().numpy()
    if rows >= 8:
        assert sure.mean() > 0.8
    assert np.array_equal(pred[sure], ref_ids[sure])
    assert np.array_equal(pred, oracle_lm_head.argmax(_bits(logits)))


def test_lm_head_wide_ties_take_lowest_index() -> None:
    g = torch.Generator(device="cuda").manual_seed(42)
    vocab, k = 20_000, 1024
    hidden, weight = _rand(g, 100, k), _rand(g, vocab, k, std=0.02)
    top = (hidden[0].float() * 0.05).to(torch.bfloat16)
    for v in (19_999, 8_000, 33, 7):  # different vocab tiles and workgroups: the lowest wins
        weight[v] = top
    announce("lm head wide ties")
    pred, logits = lm_head.lm_head_argmax(hidden, gemm.pack_weight(weight), return_logits=True)
    torch.cuda.synchronize()
    assert int(pred[0]) == 7
    assert np.array_equal(pred.cpu().numpy(), oracle_lm_head.argmax(_bits(logits)))


@pytest.mark.parametrize("rows,vocab,k", [(256, 151_936, 2048), (200, 20_000 + 24, 1024), (129, 1000 + 8, 512)])
def test_lm_head_256_rows_match_smaller_launches(rows, vocab, k) -> None:
    """129..256 token rows (8 token tiles per wave) give, row for row, the same bf16 logits and ids as
    two launches of half the rows (2 or 4 token tiles per wave): every launch sums each logit over k in
    the same order of 32x32x16 products.  Vocab sizes that leave a partial last tile and workgroups
    whose last group has fewer tiles than waves; hidden 512, 1024 and 2048."""
    g = torch.Generator(device="cuda").manual_seed(rows + vocab)
    hidden, weight = _rand(g, rows, k), _rand(g, vocab, k, std=0.02)
    weight[vocab - 1] = (hidden[rows - 1].float() * 0.05).to(torch.bfloat16)  # last row's max in the last tile
    packed = gemm.pack_weight(weight)
    half = rows // 2
    announce("lm head 256 rows vs halves", rows, vocab, k)
    pred, logits = lm_head.lm_head_argmax(hidden, packed, return_logits=True)
    pa, la = lm_head.lm_head_argmax(hidden[:half].contiguous(), packed, return_logits=True)
    pb, lb = lm_head.lm_head_argmax(hidden[half:].contiguous(), packed, return_logits=True)
    torch.cuda.synchronize()
    assert int(pred[rows - 1]) == vocab - 1
    assert torch.equal(logits.view(torch.int16), torch.cat([la, lb]).view(torch.int16))
    assert torch.equal(pred, torch.cat([pa, pb]))
    assert np.array_equal(pred.cpu().numpy(), oracle_lm_head.argmax(_bits(logits)))


def test_lm_head_256_rows_ties_take_lowest_index() -> None:
    g = torch.Generator(device="cuda").manual_seed(43)
    vocab, k = 20_000, 1024
    hidden, weight = _rand(g, 256, k), _rand(g, vocab, k, std=0.02)
    top = (hidden[200].float() * 0.05).to(torch.bfloat16)
    for v in (19_999, 8_000, 33, 7):  # different vocab tiles, waves and workgroups: the lowest wins
        weight[v] = top
    announce("lm head 256 rows ties")
    pred, logits = lm_head.lm_head_argmax(hidden, gemm.pack_weight(weight), return_logits=True)
    torch.cuda.synchronize()
    assert int(pred[200]) == 7
    assert np.array_equal(pred.cpu().numpy(), oracle_lm_head.argmax(_bits(logits)))


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


@pytest.mark.parametrize("m,k,n,epi", [(72, 2048, 4096, "store"), (80, 2048, 6144, "silu"), (256, 2048, 2048, "partial"),
                                       (129, 6144, 2048, "partial"), (200, 512, 256, "store"), (72, 2048, 2048, "add")])
def test_many_rows_equal_64_row_slices(m: int, k: int, n: int, epi: str) -> None:
    """More than 64 token rows in one call (72 = the reference's default verify width at B=8, up to
    256 for the decode step): packed rows in, packed rows out, bit-identical to the same rows
    computed 64 at a time with row-major operands (per-row arithmetic does not depend on the
    other rows).  Partials land at their rows of the [splits, m, n] array."""
    g = torch.Generator(device="cuda").manual_seed(7 * m + k + n)
    x = _rand(g, m, k)
    w = gemm.pack_weight(_rand(g, 2 * n if epi == "silu" else n, k, std=0.02))
    xp = gemm.pack_weight(x)
    announce("many rows", m, k, n, epi)
    if epi == "partial":
        splits = gemm.partial_splits(n, k)
        full = torch.full((splits, m, n), float("nan"), device="cuda")
        gemm.linear_partial(xp, w, full)
        for r0 in range(0, m, 64):
            rows = min(64, m - r0)
            part = torch.full((splits, rows, n), float("nan"), device="cuda")
            gemm.linear_partial(x[r0 : r0 + rows].contiguous(), w, part)
            torch.cuda.synchronize()
            assert torch.equal(full[:, r0 : r0 + rows].view(torch.int32), part.view(torch.int32)), r0
        return
    if epi == "add":
        r = _rand(g, m, n)
        full = r.clone()
        gemm.linear_add_(full, xp.unpack(), w)  # row-major x, one call of all m rows
        want = torch.cat([gemm.linear_add_(r[r0 : r0 + 64].clone(), x[r0 : r0 + 64], w) for r0 in range(0, m, 64)])
        torch.cuda.synchronize()
        assert torch.equal(full.view(torch.int16), want.view(torch.int16))
        return
    fn = gemm.linear if epi == "store" else gemm.linear_silu_mul
    full = fn(xp, w, out=gemm.packed_rows(m, n, "cuda")).unpack()
    want = torch.cat([fn(x[r0 : r0 + 64].contiguous(), w) for r0 in range(0, m, 64)])
    torch.cuda.synchronize()
    assert torch.equal(full.view(torch.int16), want.view(torch.int16))
