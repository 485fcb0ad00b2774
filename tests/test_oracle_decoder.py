"""Pins of ``oracle/decoder.py``, the CPU restatement of the verify forward (no GPU).

1. Golden vectors written by the reference's own ``LanguageModel.extend``
   (tests/golden/make_golden_decoder.py): hidden states, the K/V rows the step writes into each
   layer's cache, bf16 logits and their argmax must match bit for bit, in both cases (GQA 4/2 at
   S=4; GQA 16/8 at the reference's default S=9, with a sequence that holds only its new tokens).
2. The same forward from the Qwen3 equations in float64 with no intermediate rounding
   (tests/unrounded_decoder.py): the bf16 oracle must sit within bf16 error of it, and a wrong GQA
   head mapping there must fall outside, so the check can tell the plausible mistakes apart.
3. The reference's invariant (tests/test_language_fused.py:250-278): extends of 4 tokens at a time
   give the same hidden states as one causal forward over the whole sequence.
4. ``verify_step``'s row assembly and acceptance on a hand-worked case (engine.py:674-737).
"""

from __future__ import annotations

import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import decoder as oracle_decoder

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import decoder_inputs as di  # noqa: E402
import unrounded_decoder as unrounded  # noqa: E402

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "decoder_extend.npz")


def _rope(c, max_positions: int) -> tuple[torch.Tensor, torch.Tensor]:
    """language.py:160-170: fp32 angles, cos/sin stored as bf16 (cast_rope)."""
    inv_freq = 1.0 / (c.rope_theta ** (torch.arange(0, c.head_dim, 2, dtype=torch.float) / c.head_dim))
    freqs = torch.outer(torch.arange(max_positions, dtype=torch.float), inv_freq)
    return freqs.cos().to(torch.bfloat16), freqs.sin().to(torch.bfloat16)


def _oracle_weights(case: dict, p: dict[str, torch.Tensor]) -> SimpleNamespace:
    c = di.config(case)
    layers = []
    for i in range(c.num_layers):
        q = f"layers.{i}."
        layers.append(SimpleNamespace(
            input_norm=p[q + "input_layernorm.weight"],
            qkv=torch.cat([p[q + "q_proj.weight"], p[q + "k_proj.weight"], p[q + "v_proj.weight"]]),
            q_norm=p[q + "q_norm.weight"], k_norm=p[q + "k_norm.weight"], o=p[q + "o_proj.weight"],
            post_norm=p[q + "post_attention_layernorm.weight"],
            gate_up=torch.cat([p[q + "gate_proj.weight"], p[q + "up_proj.weight"]]), down=p[q + "down_proj.weight"],
        ))
    cos, sin = _rope(c, case["max_positions"])
    return SimpleNamespace(embed=p["embed_tokens.weight"], layers=layers, final_norm=p["norm.weight"],
                           lm_head=p["lm_head.weight"], rope_cos=cos, rope_sin=sin)


class _one_thread:
    """The golden vectors were written with one torch thread; CPU GEMM bits may depend on the split."""

    def __enter__(self):
        self.saved = torch.get_num_threads()
        torch.set_num_threads(1)

    def __exit__(self, *exc):
        torch.set_num_threads(self.saved)


def _run_case(name: str):
    case = di.CASES[name]
    c = di.config(case)
    params = di.parameters(case)
    inputs = di.step_inputs(case)
    k_cache, v_cache = di.caches(inputs)
    assert str(GOLDEN[f"{name}/checksum"]) == di.checksum(params, k_cache, v_cache), "regenerated inputs differ"
    for key in ("ids", "positions", "slots", "seq_lens", "table"):
        assert np.array_equal(GOLDEN[f"{name}/{key}"], inputs[key]), key
    w = _oracle_weights(case, params)
    with _one_thread():
        hidden = oracle_decoder.extend(c, w, torch.from_numpy(inputs["ids"]), torch.from_numpy(inputs["positions"]),
                                       torch.from_numpy(inputs["slots"]), torch.from_numpy(inputs["seq_lens"]),
                                       torch.from_numpy(inputs["table"]), case["tokens_per_seq"], k_cache, v_cache)
        logits = oracle_decoder.logits(w, hidden)
    return case, c, params, inputs, w, hidden, logits, k_cache, v_cache


@pytest.mark.parametrize("name", sorted(di.CASES))
def test_extend_matches_reference_vectors(name) -> None:
    case, c, _, inputs, _, hidden, logits, k_cache, v_cache = _run_case(name)
    assert np.array_equal(di.bits(hidden), GOLDEN[f"{name}/hidden"])
    assert np.array_equal(di.bits(logits), GOLDEN[f"{name}/logits"])
    assert np.array_equal(logits.argmax(-1).numpy(), GOLDEN[f"{name}/predicted"])
    flat = (c.num_layers, -1, c.num_kv_heads, c.head_dim)
    slots = torch.from_numpy(inputs["slots"])
    assert np.array_equal(di.bits(k_cache.view(flat)[:, slots]), GOLDEN[f"{name}/k_rows"])
    assert np.array_equal(di.bits(v_cache.view(flat)[:, slots]), GOLDEN[f"{name}/v_rows"])


def _rel_rms(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double(), b.double()
    return ((a - b).pow(2).sum() / b.pow(2).sum()).sqrt().item()


@pytest.mark.parametrize("name", sorted(di.CASES))
def test_extend_within_bf16_error_of_float64_equations(name) -> None:
    case, c, params, inputs, w, hidden, logits, k_cache, v_cache = _run_case(name)
    k0, v0 = di.caches(inputs)
    run = lambda **kw: unrounded.extend(c, w, inputs["ids"], inputs["positions"], inputs["seq_lens"], inputs["table"],
                                        case["tokens_per_seq"], k0, v0, di.BLOCK_SIZE, **kw)
    new_kv = []
    want = run(new_kv=new_kv)
    # bf16 activations (8 significant bits) through two layers: about 1% relative RMS.
    err = _rel_rms(hidden, want)
    assert err < 0.02, err
    flat = (c.num_layers, -1, c.num_kv_heads, c.head_dim)
    slots = torch.from_numpy(inputs["slots"])
    assert _rel_rms(k_cache.view(flat)[:, slots], torch.stack([k for k, _ in new_kv])) < 0.02
    assert _rel_rms(v_cache.view(flat)[:, slots], torch.stack([v for _, v in new_kv])) < 0.02
    # The same check tells a wrong q-head -> kv-head mapping (h % KV instead of h // G) apart.
    wrong = run(kv_head_of=lambda h: h % c.num_kv_heads)
    assert _rel_rms(hidden, wrong) > 5 * err


def test_chunked_extends_equal_one_full_forward() -> None:
    """tests/test_language_fused.py:250-278 on the oracle: 4-token extends over an empty cache give
    the hidden states one causal forward over all 12 tokens gives at the last 4 positions."""
    case = di.CASES["gqa4_s4"]
    c = di.config(case)
    params = di.parameters(case)
    w = _oracle_weights(case, params)
    b, s, n = 2, 4, 12
    table = np.array([[3], [6]], dtype=np.int32)
    tokens = np.random.default_rng(5).integers(0, c.vocab_size, size=(b, n)).astype(np.int64)
    shape = (c.num_layers, 8, di.BLOCK_SIZE, c.num_kv_heads, c.head_dim)

    def run(ck, cv, start, width):
        pos = np.concatenate([np.arange(start, start + width)] * b)
        slots = table[np.repeat(np.arange(b), width), 0].astype(np.int64) * di.BLOCK_SIZE + pos
        return oracle_decoder.extend(c, w, torch.from_numpy(tokens[:, start : start + width].reshape(-1)),
                                     torch.from_numpy(pos), torch.from_numpy(slots),
                                     torch.full((b,), start + width, dtype=torch.int32), torch.from_numpy(table), width,
                                     ck, cv)

    ck, cv = torch.zeros(shape, dtype=torch.bfloat16), torch.zeros(shape, dtype=torch.bfloat16)
    for start in range(0, n, s):
        chunked = run(ck, cv, start, s)
    fk, fv = torch.zeros_like(ck), torch.zeros_like(cv)
    full = run(fk, fv, 0, n).view(b, n, -1)[:, -s:].reshape(b * s, -1)
    # Same operations on the same values up to the GEMM's row blocking: bf16 rounding only.
    assert _rel_rms(chunked, full) < 5e-3
    assert (chunked.float() - full.float()).abs().max().item() < 0.1
    # The caches end up holding the same rows (each written once, by either path).
    assert _rel_rms(ck[:, 3, :n], fk[:, 3, :n]) < 5e-3


def test_verify_step_rows_and_acceptance_hand_case() -> None:
    """engine.py:674-737 with graph width S = k + 1: row = [last, *draft, 0 pad], positions
    length + j, slots through the table; accept = longest matching prefix + the model's token."""
    case = di.CASES["gqa4_s4"]
    c = di.config(case)
    w = _oracle_weights(case, di.parameters(case))
    histories = [[7, 8, 9, 7, 8], [1, 2, 3, 4]]  # first: suffix (7, 8) seen at 0 -> draft [9, 7, 8]; second: none
    seq_lens = np.array([40, 300], dtype=np.int32)
    table = np.array([[2, 0], [4, 5]], dtype=np.int32)
    k0 = torch.zeros(c.num_layers, 8, di.BLOCK_SIZE, c.num_kv_heads, c.head_dim, dtype=torch.bfloat16)
    seen = {}
    real_extend = oracle_decoder.extend

    def spy(config, weights, ids, positions, slots, seq_lens_, block_table, s, *rest, **kw):
        seen.update(ids=ids.tolist(), positions=positions.tolist(), slots=slots.tolist(), seq_lens=seq_lens_.tolist())
        return real_extend(config, weights, ids, positions, slots, seq_lens_, block_table, s, *rest, **kw)

    oracle_decoder.extend = spy
    try:
        drafts, predicted, taken, new_lens, _ = oracle_decoder.verify_step(c, w, histories, seq_lens, table, 3, 4,
                                                                           k0, k0.clone(), di.BLOCK_SIZE)
    finally:
        oracle_decoder.extend = real_extend
    assert drafts == [[9, 7, 8], []]
    assert seen["ids"] == [8, 9, 7, 8, 4, 0, 0, 0]
    assert seen["positions"] == [40, 41, 42, 43, 300, 301, 302, 303]
    assert seen["slots"] == [2 * 256 + 40, 2 * 256 + 41, 2 * 256 + 42, 2 * 256 + 43] + [5 * 256 + 44 + j for j in range(4)]
    assert seen["seq_lens"] == [44, 304]
    pred = predicted.tolist()
    a = 0
    while a < 3 and pred[0][a] == drafts[0][a]:
        a += 1
    assert taken[0] == drafts[0][:a] + [pred[0][a]] and taken[1] == [pred[1][0]]
    assert new_lens == [40 + a + 1, 301]
