"""Pins the fused q/k norm + RoPE + KV-write oracle (oracle/norm_rope.py).

- Golden vectors written by the reference function itself (tests/golden/make_golden.py):
  a verify-sized case, a need_kv case and tokens chosen so that the sum-of-squares order
  changes the result; the oracle matches all of them bit for bit, and an oracle with a
  different addition order (planted here, on the CPU) fails the order case.
- torch's CPU rsqrt (what the reference calls, kernels.py:145) equals float32 1/sqrt.
- Closed-form special cases: heads of constant magnitude 2^e normalise to exactly +-1, so
  with cos=1, sin=0 the output is +-w; with cos=0, sin=1 the halves swap with the sign of
  NeoX rotation.
- Error against a float64 evaluation stays within the bf16 rounding budget.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import bf16, norm_rope

GOLDEN = Path(__file__).resolve().parent / "golden" / "qk_norm_rope_store.npz"


def _case(z, name: str) -> dict:
    return {key.split("/", 1)[1]: z[key] for key in z.files if key.startswith(name + "/")}


def _run_oracle(c: dict, heads) -> tuple:
    H, KV, D = (int(x) for x in heads)
    nb, bs = int(c["num_blocks"]), int(c["block_size"])
    kc = np.full((nb, bs, KV, D), c["sentinel"][0], dtype=np.uint16)
    vc = kc.copy()
    out = norm_rope.qk_norm_rope_store(
        c["qkv"], c["q_weight"], c["k_weight"], c["cos"], c["sin"], float(c["eps"]), kc, vc, c["slots"], H, KV, D,
        need_kv=bool(c["need_kv"]),
    )
    return out, kc, vc


@pytest.mark.parametrize("name", ["verify", "prefill", "order"])
def test_oracle_matches_reference_golden_vectors(name: str) -> None:
    z = np.load(GOLDEN)
    c = _case(z, name)
    (q, k, v), kc, vc = _run_oracle(c, z["meta/heads"])
    assert np.array_equal(q, c["q_out"])
    assert np.array_equal(kc, c["k_cache_out"])
    assert np.array_equal(vc, c["v_cache_out"])
    if bool(c["need_kv"]):
        assert np.array_equal(k, c["k_out"]) and np.array_equal(v, c["v_out"])


def test_planted_sequential_sum_fails_order_vectors(monkeypatch) -> None:
    """The order case detects a different addition order: a sequential float32 sum is planted
    in the oracle and must disagree with the reference's vectors."""

    def sequential(x):
        acc = np.zeros(x.shape[:-1], dtype=np.float32)
        for i in range(x.shape[-1]):
            acc = (acc + x[..., i] * x[..., i]).astype(np.float32)
        return acc

    monkeypatch.setattr(norm_rope, "sum_squares", sequential)
    z = np.load(GOLDEN)
    c = _case(z, "order")
    (q, _, _), _, _ = _run_oracle(c, z["meta/heads"])
    assert not np.array_equal(q, c["q_out"])


def test_torch_cpu_rsqrt_is_float32_one_over_sqrt() -> None:
    g = torch.Generator().manual_seed(0)
    x = torch.cat((torch.rand(3_000_000, generator=g) * 8, torch.exp(torch.randn(3_000_000, generator=g) * 8)))
    want = np.float32(1.0) / np.sqrt(x.numpy())
    assert np.array_equal(torch.rsqrt(x).numpy(), want)


def _constant_heads(rng, n, heads, exponent):
    signs = rng.choice(np.array([-1.0, 1.0], dtype=np.float32), size=(n, heads, 128))
    return bf16.from_f32(signs * np.float32(2.0**exponent)), signs


def test_identity_rotation_gives_signed_weight() -> None:
    rng = np.random.default_rng(0)
    for exponent in (-6, 0, 5):
        x, signs = _constant_heads(rng, 3, 4, exponent)
        w = bf16.from_f32(rng.uniform(0.5, 1.5, size=128).astype(np.float32))
        cos = bf16.from_f32(np.ones((3, 64), dtype=np.float32))
        sin = bf16.from_f32(np.zeros((3, 64), dtype=np.float32))
        out = bf16.to_f32(norm_rope.norm_rope(x, w, cos, sin, eps=0.0))
        assert np.array_equal(out, signs * bf16.to_f32(w))


def test_quarter_turn_swaps_halves_with_neox_sign() -> None:
    rng = np.random.default_rng(1)
    x, signs = _constant_heads(rng, 2, 3, 1)
    w = bf16.from_f32(rng.uniform(0.5, 1.5, size=128).astype(np.float32))
    cos = bf16.from_f32(np.zeros((2, 64), dtype=np.float32))
    sin = bf16.from_f32(np.ones((2, 64), dtype=np.float32))
    out = bf16.to_f32(norm_rope.norm_rope(x, w, cos, sin, eps=0.0))
    y = signs * bf16.to_f32(w)
    assert np.array_equal(out[..., :64], -y[..., 64:])  # y1*c - y2*s with c=0, s=1
    assert np.array_equal(out[..., 64:], y[..., :64])   # y1*s + y2*c


def test_error_against_float64_within_bf16_budget() -> None:
    rng = np.random.default_rng(2)
    n, heads = 64, 8
    x = bf16.from_f32((rng.standard_normal((n, heads, 128)) * np.exp(rng.standard_normal((1, heads, 1)))).astype(np.float32))
    w = bf16.from_f32(rng.uniform(0.5, 1.5, size=128).astype(np.float32))
    angle = rng.uniform(0, 100, size=(n, 64))
    cos, sin = bf16.from_f32(np.cos(angle).astype(np.float32)), bf16.from_f32(np.sin(angle).astype(np.float32))
    got = bf16.to_f32(norm_rope.norm_rope(x, w, cos, sin, eps=1e-6)).astype(np.float64)
    h = bf16.to_f32(x).astype(np.float64)
    y = bf16.to_f32(w).astype(np.float64) * h / np.sqrt((h * h).mean(-1, keepdims=True) + 1e-6)
    c, s = bf16.to_f32(cos).astype(np.float64)[:, None], bf16.to_f32(sin).astype(np.float64)[:, None]
    truth = np.concatenate((y[..., :64] * c - y[..., 64:] * s, y[..., :64] * s + y[..., 64:] * c), -1)
    # Three bf16 roundings of values bounded by |w| * |h|/rms * sqrt(2): a few bf16 ulps of ~8.
    assert np.abs(got - truth).max() < 0.15
    assert np.abs(got - truth).mean() < 5e-3
