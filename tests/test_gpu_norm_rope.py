"""gfx950 fused q/k norm + RoPE + paged KV write vs the reference's golden vectors and the oracle.

Bit-exact on q, on the K/V written at each slot and, for need_kv, on the contiguous k/v;
every slot not written keeps its sentinel (as tests/test_kernels.py:62-65 of the reference).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import announce, pkg
from oracle import norm_rope

pytestmark = pytest.mark.gpu
kernels = pkg("kernels")
workloads = pkg("workloads")
GOLDEN = Path(__file__).resolve().parent / "golden" / "qk_norm_rope_store.npz"


def _dev(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("name", ["verify", "prefill", "order"])
def test_matches_reference_golden_vectors(name: str) -> None:
    z = np.load(GOLDEN)
    c = {key.split("/", 1)[1]: z[key] for key in z.files if key.startswith(name + "/")}
    H, KV, D = (int(x) for x in z["meta/heads"])
    nb, bs = int(c["num_blocks"]), int(c["block_size"])
    announce("golden", name, "n", c["qkv"].shape[0])
    kc = _dev(np.full((nb, bs, KV, D), c["sentinel"][0], dtype=np.uint16))
    vc = kc.clone()
    need_kv = bool(c["need_kv"])
    q, k, v = kernels.qk_norm_rope_store(
        _dev(c["qkv"]), _dev(c["q_weight"]), _dev(c["k_weight"]), _dev(c["cos"]), _dev(c["sin"]), float(c["eps"]),
        kc, vc, torch.from_numpy(c["slots"]).cuda(), H, KV, D, need_kv=need_kv,
    )
    torch.cuda.synchronize()
    assert np.array_equal(_bits(q), c["q_out"])
    assert np.array_equal(_bits(kc), c["k_cache_out"])
    assert np.array_equal(_bits(vc), c["v_cache_out"])
    if need_kv:
        assert np.array_equal(_bits(k), c["k_out"]) and np.array_equal(_bits(v), c["v_out"])
    else:
        assert k is None and v is None


def _run_case(n: int, H: int, KV: int, num_blocks: int, block_size: int, seed: int, need_kv: bool,
              slots: np.ndarray, positions: np.ndarray) -> None:
    rng = np.random.default_rng(seed)
    D = 128
    scale = np.exp(rng.standard_normal((1, H + 2 * KV, 1))).astype(np.float32)
    qkv = (rng.standard_normal((n, H + 2 * KV, D)).astype(np.float32) * scale).reshape(n, -1)
    qkv_t = torch.from_numpy(qkv).to(torch.bfloat16).cuda()
    qw = torch.from_numpy(rng.uniform(0.5, 1.5, D).astype(np.float32)).to(torch.bfloat16).cuda()
    kw = torch.from_numpy(rng.uniform(0.5, 1.5, D).astype(np.float32)).to(torch.bfloat16).cuda()
    cos_tab, sin_tab = norm_rope.rope_tables(int(positions.max()) + 1)
    cos, sin = _dev(cos_tab[positions]), _dev(sin_tab[positions])
    sentinel = 9.0
    kc = torch.full((num_blocks, block_size, KV, D), sentinel, dtype=torch.bfloat16, device="cuda")
    vc = torch.full_like(kc, sentinel)
    slots_t = torch.from_numpy(slots).cuda()
    q, k, v = kernels.qk_norm_rope_store(qkv_t, qw, kw, cos, sin, 1e-6, kc, vc, slots_t, H, KV, D, need_kv=need_kv)
    torch.cuda.synchronize()

    small_k = np.zeros((n, 1, KV, D), dtype=np.uint16)
    small_v = np.zeros_like(small_k)
    wq, wk, wv = norm_rope.qk_norm_rope_store(
        _bits(qkv_t), _bits(qw), _bits(kw), cos_tab[positions], sin_tab[positions], 1e-6, small_k, small_v,
        np.arange(n), H, KV, D, need_kv=True,
    )
    assert np.array_equal(_bits(q), wq), int((_bits(q) != wq).sum())
    flat_k, flat_v = kc.view(-1, KV, D), vc.view(-1, KV, D)
    assert np.array_equal(_bits(flat_k[slots_t]), small_k.reshape(n, KV, D))
    assert np.array_equal(_bits(flat_v[slots_t]), small_v.reshape(n, KV, D))
    if need_kv:
        assert np.array_equal(_bits(k), wk) and np.array_equal(_bits(v), wv)
    untouched = torch.ones(flat_k.shape[0], dtype=torch.bool, device="cuda")
    untouched[slots_t] = False
    assert bool((flat_k[untouched] == sentinel).all()) and bool((flat_v[untouched] == sentinel).all())


def test_config2_verify_batch_bit_exact() -> None:
    """32 sequences x 4 tokens, 16/8 heads, contexts U{256..4096}, block 16, 65,536-block pool."""
    rng = np.random.default_rng(20)
    batch = workloads.paged_batch(rng, 32, 4, (256, 4096), block_size=16, num_blocks=65_536)
    announce("config2", "n", 128)
    _run_case(128, 16, 8, 65_536, 16, seed=21, need_kv=False, slots=batch.slots, positions=batch.positions)


def test_prefill_sized_bit_exact_with_kv() -> None:
    """4,096 tokens to shuffled slots, need_kv=True (the reference GPU test's shape)."""
    rng = np.random.default_rng(22)
    slots = rng.permutation(17 * 256)[:4096].astype(np.int64)
    positions = rng.integers(0, 40960, size=4096).astype(np.int64)
    announce("prefill", "n", 4096)
    _run_case(4096, 16, 8, 17, 256, seed=23, need_kv=True, slots=slots, positions=positions)


def test_odd_head_counts_and_single_token() -> None:
    """Head counts whose 16-lane groups straddle waves (H=5, KV=3) and n=1."""
    rng = np.random.default_rng(24)
    for n in (1, 7):
        slots = rng.permutation(64)[:n].astype(np.int64)
        positions = rng.integers(0, 500, size=n).astype(np.int64)
        announce("odd heads", n)
        _run_case(n, 5, 3, 4, 16, seed=25 + n, need_kv=True, slots=slots, positions=positions)


def test_out_of_range_slot_is_not_written() -> None:
    rng = np.random.default_rng(26)
    n, H, KV, D = 3, 2, 1, 128
    qkv = torch.from_numpy(rng.standard_normal((n, (H + 2 * KV) * D)).astype(np.float32)).to(torch.bfloat16).cuda()
    w = torch.ones(D, dtype=torch.bfloat16, device="cuda")
    cos = torch.ones(n, 64, dtype=torch.bfloat16, device="cuda")
    sin = torch.zeros_like(cos)
    kc = torch.full((2, 4, KV, D), 9.0, dtype=torch.bfloat16, device="cuda")
    vc = kc.clone()
    slots = torch.tensor([1, -1, 8], dtype=torch.int64, device="cuda")  # only slot 1 is inside 2*4 slots
    announce("slot bounds")
    kernels.qk_norm_rope_store(qkv, w, w, cos, sin, 1e-6, kc, vc, slots, H, KV, D, need_kv=False)
    torch.cuda.synchronize()
    flat = kc.view(-1, KV, D)
    assert not bool((flat[1] == 9.0).all())
    keep = [i for i in range(8) if i != 1]
    assert bool((flat[keep] == 9.0).all()) and bool((vc.view(-1, KV, D)[keep] == 9.0).all())

