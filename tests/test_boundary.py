"""The drop-in boundary refuses CPU tensors instead of falling back to a CPU path
(the reference dispatches CPU tensors to torch code, kernels.py:111-112; this build
has none), and validates shapes on the host before any launch."""

from __future__ import annotations

import pytest
import torch

from conftest import pkg

kernels = pkg("kernels")
spec = pkg("speculative")


def _bf(*shape):
    return torch.zeros(*shape, dtype=torch.bfloat16)


def test_qk_norm_rope_store_rejects_cpu_tensors() -> None:
    w = _bf(128)
    with pytest.raises(RuntimeError, match="GPU"):
        kernels.qk_norm_rope_store(_bf(1, 4 * 128), w, w, _bf(1, 64), _bf(1, 64), 1e-6, _bf(1, 1, 1, 128),
                                   _bf(1, 1, 1, 128), torch.zeros(1, dtype=torch.long), 2, 1, 128, need_kv=False)


def test_speculative_rejects_cpu_tensors() -> None:
    h = torch.zeros(2, 8, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        spec.propose_batch(h, torch.zeros(2, dtype=torch.int32), 3)


language = pkg("language")


def _rows(t, dtype):
    return torch.zeros(t, dtype=dtype)


def test_extend_batch_takes_the_reference_positional_form() -> None:
    """ExtendBatch(embeds, positions, slots, seq_lens, block_table, S) as engine.py:716-724 builds it;
    DecodeBatch(embeds, positions, slots, seq_lens, block_table) as engine.py:594-600."""
    emb = _bf(8, 64)
    eb = language.ExtendBatch(emb, _rows(8, torch.int64), _rows(8, torch.int64), _rows(2, torch.int32),
                              torch.zeros(2, 3, dtype=torch.int32), 4)
    assert eb.embeds is emb and eb.ids is None and eb.tokens_per_seq == 4
    db = language.DecodeBatch(_bf(2, 64), _rows(2, torch.int64), _rows(2, torch.int64), _rows(2, torch.int32),
                              torch.zeros(2, 3, dtype=torch.int32))
    assert db.as_extend().embeds is db.embeds and db.as_extend().tokens_per_seq == 1
    ids = _rows(8, torch.int64)
    eb = language.ExtendBatch(None, _rows(8, torch.int64), _rows(8, torch.int64), _rows(2, torch.int32),
                              torch.zeros(2, 3, dtype=torch.int32), 4, ids=ids)
    assert eb.ids is ids and eb.embeds is None


@pytest.mark.parametrize("kind", ["extend", "decode"])
def test_batches_reject_ids_of_the_wrong_type(kind: str) -> None:
    """A bf16 tensor given as ids (or token ids given as embeds) raises instead of being gathered as
    clamped garbage; so does giving both or neither."""
    rest = (_rows(8, torch.int64), _rows(8, torch.int64), _rows(2, torch.int32), torch.zeros(2, 3, dtype=torch.int32))
    make = (lambda e, **kw: language.ExtendBatch(e, *rest, 4, **kw)) if kind == "extend" else \
        (lambda e, **kw: language.DecodeBatch(e, *rest, **kw))
    with pytest.raises(TypeError, match="ids must be int64"):
        make(None, ids=_bf(8))
    with pytest.raises(TypeError, match="ids="):
        make(_rows(8, torch.int64))
    with pytest.raises(TypeError, match="bf16"):
        make(torch.zeros(8, 64, dtype=torch.float32))
    with pytest.raises(ValueError, match="either"):
        make(_bf(8, 64), ids=_rows(8, torch.int64))
    with pytest.raises(ValueError, match="either"):
        make(None)


def test_embed_tokens_rejects_float_ids() -> None:
    with pytest.raises(TypeError, match="int64 or int32"):
        language.LanguageModel.embed_tokens(None, _bf(4))


def test_ngram_extend_refuses_a_gap_in_the_index() -> None:
    """NgramProposer.extend(tokens, old_length) past the indexed length would leave positions the
    reference's dict never gets (speculative.py:28-31) and the device prefix index cannot skip:
    refused before anything is launched."""
    proposer = object.__new__(spec.NgramProposer)
    proposer._indexed = 10
    with pytest.raises(ValueError, match="unindexed"):
        proposer.extend(list(range(20)), 15)
