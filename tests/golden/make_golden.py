"""Write golden vectors for the fused q/k RMSNorm + RoPE + KV write from the reference itself.

Runs ``qk_norm_rope_store_reference`` of the reference (oxr_runtime/kernels.py:133-165,
the function its CPU path dispatches to at kernels.py:111-112) on seeded inputs and
stores inputs and outputs as raw bf16 bits in ``qk_norm_rope_store.npz``.  This is the
one function on the path whose exact bits (torch's CPU rsqrt and bf16 rounding) no
closed form in the reference's tests pins, so its vectors come from the reference.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden.py /root/reference

The committed .npz is data: inputs and expected outputs, nothing from the reference's
source.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "qk_norm_rope_store.npz"


def _bits(t):
    import torch

    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def main(reference_root: str) -> None:
    import torch

    sys.path.insert(0, reference_root)
    from oxr_runtime import kernels  # noqa: PLC0415  (the reference module)

    H, KV, D, BLOCK = 16, 8, 128, 16
    cases = {}
    for name, n, need_kv, seed in (("verify", 32, False, 1), ("prefill", 12, True, 2)):
        g = torch.Generator().manual_seed(seed)
        # Per-head magnitude spread so the sum of squares exercises many exponents.
        scale = torch.exp(torch.randn(1, H + 2 * KV, 1, generator=g))
        qkv = (torch.randn(n, H + 2 * KV, D, generator=g) * scale).to(torch.bfloat16).reshape(n, -1).contiguous()
        qw = (0.5 + torch.rand(D, generator=g)).to(torch.bfloat16)
        kw = (0.5 + torch.rand(D, generator=g)).to(torch.bfloat16)
        # RoPE tables exactly as language.py:160-170 builds them, theta = 1e6.
        inv_freq = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float) / D))
        positions = torch.randint(0, 4096, (n,), generator=g)
        freqs = torch.outer(positions.float(), inv_freq)
        cos, sin = freqs.cos().to(torch.bfloat16), freqs.sin().to(torch.bfloat16)
        num_blocks = 8
        slots = torch.randperm(num_blocks * BLOCK, generator=g)[:n].long()
        sentinel = torch.tensor(9.0).to(torch.bfloat16)
        k_cache = torch.full((num_blocks, BLOCK, KV, D), 9.0).to(torch.bfloat16)
        v_cache = torch.full((num_blocks, BLOCK, KV, D), 9.0).to(torch.bfloat16)
        q, k, v = kernels.qk_norm_rope_store_reference(
            qkv, qw, kw, cos, sin, 1e-6, k_cache, v_cache, slots, H, KV, D, need_kv=need_kv
        )
        case = {
            "qkv": _bits(qkv), "q_weight": _bits(qw), "k_weight": _bits(kw), "cos": _bits(cos), "sin": _bits(sin),
            "positions": positions.numpy().astype(np.int64), "slots": slots.numpy().astype(np.int64),
            "num_blocks": np.int64(num_blocks), "block_size": np.int64(BLOCK), "sentinel": _bits(sentinel.reshape(1)),
            "need_kv": np.bool_(need_kv), "eps": np.float32(1e-6),
            "q_out": _bits(q), "k_cache_out": _bits(k_cache), "v_cache_out": _bits(v_cache),
        }
        if need_kv:
            case["k_out"], case["v_out"] = _bits(k), _bits(v)
        for key, value in case.items():
            cases[f"{name}/{key}"] = value
    # Tokens on which the sum-of-squares order matters: heads with a wide spread of element
    # magnitudes, kept only where a plain mean(h^2) (another order) changes the bf16 output, so a
    # kernel with any other addition order fails these vectors.
    g = torch.Generator().manual_seed(3)
    n_try = 4096
    wide = torch.randn(n_try, H + 2 * KV, D, generator=g) * torch.exp(3 * torch.randn(n_try, H + 2 * KV, D, generator=g))
    qkv = wide.to(torch.bfloat16).reshape(n_try, -1).contiguous()
    qw = (0.5 + torch.rand(D, generator=g)).to(torch.bfloat16)
    kw = (0.5 + torch.rand(D, generator=g)).to(torch.bfloat16)
    cos = torch.ones(n_try, D // 2).to(torch.bfloat16)
    sin = torch.zeros(n_try, D // 2).to(torch.bfloat16)
    caches = [torch.zeros(n_try, 1, KV, D).to(torch.bfloat16) for _ in range(2)]
    slots = torch.arange(n_try).long()
    q, _, _ = kernels.qk_norm_rope_store_reference(qkv, qw, kw, cos, sin, 1e-6, *caches, slots, H, KV, D, need_kv=False)
    h = qkv.view(n_try, H + 2 * KV, D)[:, :H].float()
    alt = (qw * (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)).to(torch.bfloat16)
    differs = (q != alt).flatten(1).any(1).nonzero().flatten()[:32]
    keep = differs.tolist()
    n = len(keep)
    sel = torch.tensor(keep)
    k_cache = torch.full((4, BLOCK, KV, D), 9.0).to(torch.bfloat16)
    v_cache = torch.full((4, BLOCK, KV, D), 9.0).to(torch.bfloat16)
    slots = torch.randperm(4 * BLOCK, generator=g)[:n].long()
    qkv_sel = qkv[sel].contiguous()
    q, _, _ = kernels.qk_norm_rope_store_reference(
        qkv_sel, qw, kw, cos[:n], sin[:n], 1e-6, k_cache, v_cache, slots, H, KV, D, need_kv=False
    )
    order = {
        "qkv": _bits(qkv_sel), "q_weight": _bits(qw), "k_weight": _bits(kw), "cos": _bits(cos[:n]),
        "sin": _bits(sin[:n]), "positions": np.zeros(n, dtype=np.int64), "slots": slots.numpy().astype(np.int64),
        "num_blocks": np.int64(4), "block_size": np.int64(BLOCK), "sentinel": _bits(torch.tensor([9.0]).to(torch.bfloat16)),
        "need_kv": np.bool_(False), "eps": np.float32(1e-6),
        "q_out": _bits(q), "k_cache_out": _bits(k_cache), "v_cache_out": _bits(v_cache),
    }
    for key, value in order.items():
        cases[f"order/{key}"] = value
    print(f"order-sensitive tokens kept: {n}")
    cases["meta/heads"] = np.array([H, KV, D], dtype=np.int64)
    np.savez_compressed(OUT, **cases)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
