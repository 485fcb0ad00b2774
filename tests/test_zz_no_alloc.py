"""The entry point that allocates nothing (oxr_qk_norm_rope_paged_extend_static) against the
one that takes a workspace (oxr_qk_norm_rope_paged_extend), through the C ABI: two calls in a
row, the second on a smaller batch and context, each bit-identical to the workspace entry point
in output and cache rows."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce, pkg

pytestmark = pytest.mark.gpu
_lib = pkg("_lib")
language = pkg("language")
attention = pkg("attention")
workloads = pkg("workloads")

H, KV, D, BS = 16, 8, 128, 16


def _case(seed: int, batch: int, ctx: tuple[int, int], num_blocks: int):
    rng = np.random.default_rng(seed)
    pb = workloads.paged_batch(rng, batch, 4, ctx, block_size=BS, num_blocks=num_blocks)
    g = torch.Generator(device="cuda").manual_seed(seed)
    kc = torch.randn(num_blocks, BS, KV, D, generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn(num_blocks, BS, KV, D, generator=g, device="cuda").to(torch.bfloat16)
    qkv = torch.randn(batch * 4, (H + 2 * KV) * D, generator=g, device="cuda").to(torch.bfloat16)
    qw = (0.5 + torch.rand(D, generator=g, device="cuda")).to(torch.bfloat16)
    kw = (0.5 + torch.rand(D, generator=g, device="cuda")).to(torch.bfloat16)
    cos, sin = language.rope_tables(language.QWEN_SYNTHETIC, 20_000)
    d = lambda a, dt: torch.from_numpy(np.asarray(a)).to(dt).cuda()
    return dict(qkv=qkv, qw=qw, kw=kw, cos=cos.cuda(), sin=sin.cuda(), pos=d(pb.positions, torch.int64),
                slots=d(pb.slots, torch.int64), seq=d(pb.seq_lens, torch.int32),
                table=d(pb.block_table, torch.int32), kc=kc, vc=vc, batch=batch,
                max_seq_len=pb.block_table.shape[1] * BS, num_blocks=num_blocks)


def _args(c, kc, vc, out):
    return (c["qkv"].data_ptr(), c["qw"].data_ptr(), c["kw"].data_ptr(), c["cos"].data_ptr(), c["sin"].data_ptr(),
            c["cos"].shape[0], c["pos"].data_ptr(), 1e-6, kc.data_ptr(), vc.data_ptr(), c["slots"].data_ptr(),
            c["num_blocks"] * BS, c["seq"].data_ptr(), c["table"].data_ptr(), c["table"].shape[1], c["batch"], 4, H,
            KV, D, BS, c["num_blocks"], c["max_seq_len"], D ** -0.5, out.data_ptr(), 0)


def test_static_scratch_matches_workspace_entry_point() -> None:
    stream = _lib.stream(torch.device("cuda"))
    for step, (seed, batch, ctx) in enumerate(((1, 8, (3000, 8000)), (2, 3, (200, 1500)))):
        c = _case(seed, batch, ctx, num_blocks=8192)
        out_ref = torch.zeros(batch, 4, H, D, dtype=torch.bfloat16, device="cuda")
        out_new = torch.full_like(out_ref, 7.0)
        k_ref, v_ref = c["kc"].clone(), c["vc"].clone()
        need = attention.workspace_bytes(batch, KV, c["max_seq_len"])
        assert need <= _lib.lib().oxr_static_scratch_bytes()
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        announce("no-alloc entry point, call", step, "batch", batch, "ctx", ctx)
        _lib.call("oxr_qk_norm_rope_paged_extend", *_args(c, k_ref, v_ref, out_ref), ws.data_ptr(), need, stream)
        _lib.call("oxr_qk_norm_rope_paged_extend_static", *_args(c, c["kc"], c["vc"], out_new), stream)
        torch.cuda.synchronize()
        assert torch.equal(out_new.view(torch.int16), out_ref.view(torch.int16))
        assert torch.equal(c["kc"].view(torch.int16), k_ref.view(torch.int16))
        assert torch.equal(c["vc"].view(torch.int16), v_ref.view(torch.int16))
