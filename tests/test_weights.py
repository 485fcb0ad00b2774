"""``LanguageWeights.from_state_dict``: the reference LanguageModel's parameter names
(language.py:155-158, 221-231), split or fused projections (language.py:234-245), into the fused
layout the gfx950 forward runs on.  CPU tensors: this is name and layout bookkeeping."""

from __future__ import annotations

import pytest
import torch

from conftest import pkg

language = pkg("language")

C = language.LanguageConfig(256, 384, 2, 4, 2, 128, 1e-6, 1e6, 300)


def _reference_state(fused: bool) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(0)
    r = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)
    h, d = C.hidden_size, C.head_dim
    st = {"embed_tokens.weight": r(C.vocab_size, h), "norm.weight": r(h), "lm_head.weight": r(C.vocab_size, h)}
    for i in range(C.num_layers):
        p = f"layers.{i}."
        st.update({p + "input_layernorm.weight": r(h), p + "post_attention_layernorm.weight": r(h),
                   p + "q_norm.weight": r(d), p + "k_norm.weight": r(d), p + "o_proj.weight": r(h, C.num_heads * d),
                   p + "down_proj.weight": r(h, C.intermediate_size)})
        q, k, v = r(C.num_heads * d, h), r(C.num_kv_heads * d, h), r(C.num_kv_heads * d, h)
        gate, up = r(C.intermediate_size, h), r(C.intermediate_size, h)
        if fused:
            st[p + "qkv_proj.weight"] = torch.cat((q, k, v))
            st[p + "gate_up_proj.weight"] = torch.cat((gate, up))
        else:
            st.update({p + "q_proj.weight": q, p + "k_proj.weight": k, p + "v_proj.weight": v,
                       p + "gate_proj.weight": gate, p + "up_proj.weight": up})
    return st


def test_split_and_fused_names_give_the_same_weights() -> None:
    split, fused = _reference_state(False), _reference_state(True)
    a = language.LanguageWeights.from_state_dict(C, split, 64)
    b = language.LanguageWeights.from_state_dict(C, fused, 64)
    for i in range(C.num_layers):
        p = f"layers.{i}."
        want_qkv = torch.cat((split[p + "q_proj.weight"], split[p + "k_proj.weight"], split[p + "v_proj.weight"]))
        assert torch.equal(a.layers[i].qkv, want_qkv) and torch.equal(b.layers[i].qkv, want_qkv)
        want_gu = torch.cat((split[p + "gate_proj.weight"], split[p + "up_proj.weight"]))
        assert torch.equal(a.layers[i].gate_up, want_gu) and torch.equal(b.layers[i].gate_up, want_gu)
        assert torch.equal(a.layers[i].down, split[p + "down_proj.weight"])
        assert torch.equal(a.layers[i].input_norm, split[p + "input_layernorm.weight"])
        assert torch.equal(a.layers[i].post_norm, split[p + "post_attention_layernorm.weight"])
    assert torch.equal(a.embed, split["embed_tokens.weight"]) and torch.equal(a.lm_head, split["lm_head.weight"])
    cos, sin = language.rope_tables(C, 64)
    assert torch.equal(a.rope_cos, cos) and torch.equal(a.rope_sin, sin)


def test_missing_unexpected_and_misshapen_parameters_raise() -> None:
    st = _reference_state(False)
    missing = dict(st)
    del missing["layers.1.k_norm.weight"]
    with pytest.raises(KeyError):
        language.LanguageWeights.from_state_dict(C, missing, 64)
    extra = dict(st, **{"layers.2.q_proj.weight": st["layers.0.q_proj.weight"]})
    with pytest.raises(KeyError):
        language.LanguageWeights.from_state_dict(C, extra, 64)
    bad = dict(st, **{"layers.0.o_proj.weight": st["layers.0.o_proj.weight"][:, :-8]})
    with pytest.raises(ValueError):
        language.LanguageWeights.from_state_dict(C, bad, 64)
