"""The one-launch MLP block (oxr_mlp_block) against the oracle's MLP and the three-launch form.

Config-5 shapes (hidden 2048, intermediate 6144, weights ~N(0, 0.02)), T token rows from 1 to 32,
o_proj arriving as 4 or 8 fp32 partial slices:
- the new residual and every XCD's copy of the normalised rows are bit-identical to what
  oxr_add_partials_rms_norm produces (the same arithmetic in the same order);
- the block's output (its 8 fp32 slices summed in slice order, rounded to bf16 as the reference's
  down_proj output) is within |err| <= 2e-2 + 1e-2 |ref| of the oracle's ``_mlp``
  (language.py:266-269: bf16 linears with fp32 accumulation, silu_mul, bf16 rounding points);
- against the three-launch form (add + RMSNorm, gate_up with the SiLU epilogue, down k-split), whose
  fp32 sums differ only in accumulation order, the outputs agree to 1e-3 of their largest value;
- the error word stays 0 (placement and every wait inside the launch held), also over calls in a
  row with different T on one workspace.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from conftest import announce, pkg
from oracle import decoder as oracle_decoder

pytestmark = pytest.mark.gpu
gemm = pkg("gemm")
mlp = pkg("mlp")

H, I = 2048, 6144
EPS = 1e-6
ATOL, RTOL = 2e-2, 1e-2


@pytest.fixture(scope="module")
def weights():
    if not mlp.supported(1, H, I):
        pytest.skip("the one-launch MLP block needs an MI355X in single-partition mode")
    g = torch.Generator(device="cuda").manual_seed(7)
    gate_up = (torch.randn(2 * I, H, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    down = (torch.randn(H, I, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    norm = (torch.rand(H, generator=g, device="cuda") + 0.5).to(torch.bfloat16)
    return dict(gate_up=gate_up, down=down, norm=norm, gate_up_packed=gemm.pack_weight(gate_up),
                gate_up_il=gemm.pack_weight(mlp.interleave_gate_up(gate_up)), down_packed=gemm.pack_weight(down))


def _inputs(t: int, splits: int, seed: int):
    g = torch.Generator(device="cuda").manual_seed(seed)
    o_part = torch.randn(splits, t, H, generator=g, device="cuda") * 0.3
    residual = torch.randn(t, H, generator=g, device="cuda").to(torch.bfloat16)
    return o_part.contiguous(), residual


def _oracle_mlp(o_part: torch.Tensor, residual: torch.Tensor, w) -> tuple[torch.Tensor, torch.Tensor]:
    """(new residual, bf16 MLP output) on the CPU, language.py:94-104, 266-269."""
    o = o_part.cpu()[0]
    for s in range(1, o_part.shape[0]):
        o = o + o_part.cpu()[s]
    res = o.to(torch.bfloat16) + residual.cpu()
    h = oracle_decoder.rms_norm(res, w["norm"].cpu(), EPS)
    gu = F.linear(h.float(), w["gate_up"].cpu().float()).to(torch.bfloat16)
    act = oracle_decoder.silu_mul(gu)
    out = F.linear(act.float(), w["down"].cpu().float()).to(torch.bfloat16)
    return res, out


def _three_launch(o_part, residual, w, t):
    res = residual.clone()
    h = gemm.packed_rows(t, H, "cuda")
    gemm.add_partials_rms_norm(o_part, o_part.shape[0], res, w["norm"], EPS, h)
    act = gemm.packed_rows(t, I, "cuda")
    gemm.linear_silu_mul(h, w["gate_up_packed"], out=act)
    part = torch.zeros(gemm.partial_splits(H, I), t, H, device="cuda")
    n = gemm.linear_partial(act, w["down_packed"], part)
    return res, h, part[:n].sum(0)


def _run_block(o_part, residual, w, ws, t):
    res_out = torch.zeros_like(residual)
    part = torch.full((mlp.SPLITS_OUT, t, H), float("nan"), device="cuda")
    mlp.mlp_block(o_part, o_part.shape[0], residual, w["norm"], EPS, w["gate_up_il"], w["down_packed"], res_out,
                  part, ws)
    out = part[0].clone()
    for s in range(1, mlp.SPLITS_OUT):
        out = out + part[s]
    return res_out, out


@pytest.mark.parametrize("t,splits", [(32, 4), (1, 4), (7, 8), (16, 4), (17, 8), (29, 4)])
def test_mlp_block_matches_oracle_and_three_launch_form(weights, t, splits) -> None:
    ws = mlp.workspace("cuda")
    o_part, residual = _inputs(t, splits, seed=100 + t)
    announce("mlp_block", f"t={t}", f"o_splits={splits}")
    res_out, out = _run_block(o_part, residual, weights, ws, t)
    torch.cuda.synchronize()
    assert mlp.error_bits(ws) == 0
    res3, h3, out3 = _three_launch(o_part, residual, weights, t)
    torch.cuda.synchronize()
    assert torch.equal(res_out, res3)
    # Every XCD's copy of the normalised rows (workspace after the 4 KiB of control words).
    copies = ws[4096: 4096 + 8 * 32 * H * 2].view(torch.bfloat16).view(8, 32 * H)
    want_h = h3.data[: ((t + 15) // 16) * 16 * H]
    for x in range(8):
        got = gemm.PackedMatrix(copies[x, : want_h.numel()].contiguous(), t, H).unpack()
        assert torch.equal(got, gemm.PackedMatrix(want_h, t, H).unpack()), f"XCD {x}"
    assert not torch.isnan(out).any()
    scale = out3.abs().max().item()
    assert (out - out3).abs().max().item() <= 1e-3 * scale, ((out - out3).abs().max().item(), scale)
    want_res, want_out = _oracle_mlp(o_part, residual, weights)
    assert torch.equal(res_out.cpu(), want_res)
    got = out.to(torch.bfloat16).float().cpu()
    err = (got - want_out.float()).abs()
    bound = ATOL + RTOL * want_out.float().abs()
    assert bool((err <= bound).all()), (err.max().item(), (err - bound).max().item())


def test_mlp_block_calls_in_a_row_reuse_the_workspace(weights) -> None:
    """The control words are left zero by each launch: a second and third call on the same workspace,
    with fewer and then more rows, are as correct as the first."""
    ws = mlp.workspace("cuda")
    for i, t in enumerate((32, 5, 24)):
        o_part, residual = _inputs(t, 4, seed=200 + i)
        announce("mlp_block in a row", f"call={i}", f"t={t}")
        res_out, out = _run_block(o_part, residual, weights, ws, t)
        res3, _, out3 = _three_launch(o_part, residual, weights, t)
        torch.cuda.synchronize()
        assert mlp.error_bits(ws) == 0
        assert torch.equal(res_out, res3)
        assert (out - out3).abs().max().item() <= 1e-3 * out3.abs().max().item()
    ctl = ws[: 4096].view(torch.int32)
    assert int(ctl.abs().sum().item()) == 0


def test_mlp_block_refuses_what_it_cannot_run(weights) -> None:
    lib = pkg("_lib").lib()
    assert not lib.oxr_mlp_block_supported(33, H, I, 4)
    assert not lib.oxr_mlp_block_supported(8, 4096, I, 4)
    assert not lib.oxr_mlp_block_supported(8, H, I, 2)
    o_part, residual = _inputs(8, 4, seed=3)
    ws = mlp.workspace("cuda")
    with pytest.raises(RuntimeError):
        mlp.mlp_block(o_part, 4, residual, weights["norm"], EPS, weights["gate_up_il"], weights["down_packed"],
                      residual, torch.zeros(8, 8, H, device="cuda"), ws)  # residual_out == residual_in
    with pytest.raises(RuntimeError):
        mlp.mlp_block(o_part, 4, residual, weights["norm"], EPS, weights["gate_up_il"], weights["down_packed"],
                      torch.zeros_like(residual), torch.zeros(8, 8, H, device="cuda"), ws[:1024])
