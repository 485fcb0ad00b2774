"""Pins the paged-attention oracle (oracle/attention.py), whose reference is the test stub of
tests/test_language_fused.py:19-57 (flash-attn itself is not in the reference tree).

- Identical keys give a uniform softmax: each new token's output is the mean of V over the
  keys it may see, which fixes the end-aligned causal mask (token i of n sees m - n + i + 1).
- Each row equals single-query attention over its visible prefix (mask alignment again).
- GQA: kv head h // (H / KV); duplicating kv heads to H changes nothing.
- One visible key returns that key's V exactly.
"""

from __future__ import annotations

import numpy as np

from oracle import attention, bf16


def test_identical_keys_average_visible_values() -> None:
    rng = np.random.default_rng(0)
    n, m, h, kv, d = 4, 9, 4, 2, 8
    q = rng.standard_normal((n, h, d))
    k = np.repeat(rng.standard_normal((1, kv, d)), m, axis=0)
    v = rng.standard_normal((m, kv, d))
    out = attention.attend(q, k, v, 0.3)
    for i in range(n):
        visible = m - n + i + 1
        for head in range(h):
            np.testing.assert_allclose(out[i, head], v[:visible, head // (h // kv)].mean(0), rtol=1e-12, atol=1e-12)


def test_rows_equal_prefix_attention() -> None:
    rng = np.random.default_rng(1)
    n, m, h, kv, d = 3, 11, 4, 4, 16
    q, k, v = rng.standard_normal((n, h, d)), rng.standard_normal((m, kv, d)), rng.standard_normal((m, kv, d))
    out = attention.attend(q, k, v, 0.25)
    for i in range(n):
        visible = m - n + i + 1
        single = attention.attend(q[i : i + 1], k[:visible], v[:visible], 0.25)
        np.testing.assert_allclose(out[i], single[0], rtol=1e-12, atol=1e-12)


def test_gqa_equals_duplicated_heads() -> None:
    rng = np.random.default_rng(2)
    n, m, h, kv, d = 2, 7, 6, 2, 8
    q, k, v = rng.standard_normal((n, h, d)), rng.standard_normal((m, kv, d)), rng.standard_normal((m, kv, d))
    rep = h // kv
    full = attention.attend(q, np.repeat(k, rep, axis=1), np.repeat(v, rep, axis=1), 0.5)
    np.testing.assert_allclose(attention.attend(q, k, v, 0.5), full, rtol=1e-12, atol=1e-12)
    # and a wrong grouping (h % kv) would differ
    wrong = attention.attend(q, np.tile(k, (1, rep, 1)), np.tile(v, (1, rep, 1)), 0.5)
    assert not np.allclose(full, wrong)


def test_single_visible_key() -> None:
    rng = np.random.default_rng(3)
    q, k, v = rng.standard_normal((1, 2, 4)), rng.standard_normal((1, 1, 4)), rng.standard_normal((1, 1, 4))
    np.testing.assert_allclose(attention.attend(q, k, v, 1.0)[0], np.repeat(v[0], 2, axis=0), rtol=1e-12)


def test_varlen_closed_forms_and_invariants() -> None:
    """varlen: (1) zero queries give every visible key the same weight, so each output row is the
    mean of the visible values (prefix mean when causal, full mean otherwise); (2) causal row i
    equals non-causal attention over the prefix [0, i]; (3) a one-token sequence returns its own
    value; (4) sequences do not see each other (a batch equals its sequences run alone)."""
    rng = np.random.default_rng(5)
    lens = [1, 5, 9]
    cu = np.concatenate([[0], np.cumsum(lens)])
    T, H, KV, D = int(cu[-1]), 4, 2, 8
    rand = lambda *shape: bf16.from_f32(rng.standard_normal(shape).astype(np.float32))
    q, k, v = rand(T, H, D), rand(T, KV, D), rand(T, KV, D)
    vf = np.repeat(bf16.to_f32(v).astype(np.float64), H // KV, axis=1)
    zero_q = np.zeros_like(q)
    causal0 = attention.varlen(zero_q, k, v, cu, 0.3, True)
    full0 = attention.varlen(zero_q, k, v, cu, 0.3, False)
    for a, b in zip(cu[:-1], cu[1:]):
        for i in range(a, b):
            np.testing.assert_allclose(causal0[i], vf[a : i + 1].mean(0), rtol=1e-12, atol=1e-12)
            np.testing.assert_allclose(full0[i], vf[a:b].mean(0), rtol=1e-12, atol=1e-12)
    causal = attention.varlen(q, k, v, cu, 0.3, True)
    qf, kf, vf32 = bf16.to_f32(q), bf16.to_f32(k), bf16.to_f32(v)
    for a, b in zip(cu[:-1], cu[1:]):
        for i in range(a, b):
            prefix = attention.attend(qf[i : i + 1], kf[a : i + 1], vf32[a : i + 1], 0.3, causal=False)
            np.testing.assert_allclose(causal[i], prefix[0], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(causal[0], vf[0], rtol=1e-12, atol=1e-12)  # the one-token sequence
    alone = attention.varlen(q[1:6], k[1:6], v[1:6], np.array([0, 5]), 0.3, True)
    np.testing.assert_allclose(causal[1:6], alone, rtol=1e-12, atol=1e-12)
