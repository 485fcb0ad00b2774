"""The oracle's bf16 conversion equals torch's CPU conversion (c10 round_to_nearest_even)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import bf16


def _torch_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_matches_torch_on_random_and_special_values() -> None:
    rng = np.random.default_rng(0)
    # Random bit patterns cover every exponent, subnormals, infinities and NaNs.
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001, 0xFFFFFFFF,
                        0x00000001, 0x007FFFFF, 0x3F808000, 0x3F818000, 0x3F807FFF, 0x7F7FFFFF], dtype=np.uint32)
    x = np.concatenate((bits, special)).view(np.float32)
    got = bf16.from_f32(x)
    want = _torch_bits(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert (got[nan] == 0x7FC0).all()
    assert (np.isnan(bf16.to_f32(want[nan]))).all()


def test_ties_round_to_even() -> None:
    # 1 + 2^-8 lies halfway between bf16 1.0 and 1.0078125: even mantissa (1.0) wins.
    halfway = np.array([1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8], dtype=np.float32)
    assert bf16.from_f32(halfway).tolist() == [0x3F80, 0x3F82]


def test_round_trip_is_exact_for_bf16_values() -> None:
    all_bits = np.arange(2**16, dtype=np.uint16)
    finite = ~np.isnan(bf16.to_f32(all_bits))
    assert np.array_equal(bf16.from_f32(bf16.to_f32(all_bits))[finite], all_bits[finite])
