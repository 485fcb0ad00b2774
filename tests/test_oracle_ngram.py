"""Pins the n-gram drafting / acceptance oracle (oracle/ngram.py).

- Known answers restated from the reference's tests (tests/test_speculative.py:8-41).
- Two independent restatements agree: the reference's dict (speculative.py:15-39) and the
  closed form "largest (m(p), p)", on thousands of random and repetitive histories, for
  several n caps and for proposers indexed on a prefix only.
- Hand cases that separate plausible mistakes: longest n beats a later shorter match;
  latest occurrence wins among equal lengths; drafts stop at the end of the history.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import pkg
from oracle import ngram

workloads = pkg("workloads")


def test_known_answer_latest_match_of_longest_suffix() -> None:
    td, end, one, two = 10, 11, 1, 2
    tokens = [td, one, end, td, two, end, td]
    assert ngram.NgramIndex(tokens).propose(tokens, 3) == [two, end, td]
    assert ngram.propose_closed_form(tokens, 3) == [two, end, td]


def test_known_answer_no_match() -> None:
    tokens = [1, 2, 3, 4]
    assert ngram.NgramIndex(tokens).propose(tokens, 8) == []
    assert ngram.propose_closed_form(tokens, 8) == []


def test_known_answer_extend_equals_rebuild() -> None:
    tokens = [5, 6, 7, 5, 6, 8, 5, 6, 7, 9, 5, 6]
    incremental = ngram.NgramIndex(tokens[:5])
    incremental.extend(tokens, 5)
    for k in (1, 2, 4):
        assert incremental.propose(tokens, k) == ngram.NgramIndex(tokens).propose(tokens, k)


def test_known_answer_accept() -> None:
    assert ngram.accept([7, 8, 9, 10], [7, 8, 3, 0, 0]) == [7, 8, 3]
    assert ngram.accept([7, 8], [7, 8, 5]) == [7, 8, 5]
    assert ngram.accept([7, 8], [1, 8, 5]) == [1]
    assert ngram.accept([], [4]) == [4]


def test_longest_suffix_beats_later_shorter_match() -> None:
    tokens = [1, 2, 3, 9, 5, 3, 8, 1, 2, 3]
    # [1,2,3] matched at p=3 (-> 9 5 3); only [3] matches later, at p=6 (-> 8 ...).
    for propose in (lambda t, k: ngram.NgramIndex(t).propose(t, k), ngram.propose_closed_form):
        assert propose(tokens, 3) == [9, 5, 3]


def test_latest_occurrence_wins_and_draft_stops_at_end() -> None:
    tokens = [4, 7, 1, 4, 7, 2, 4, 7]
    # [4,7] at p=2 and p=5: the later one proposes 2 4 7; with k=5 it stops at the end.
    assert ngram.propose_closed_form(tokens, 5) == [2, 4, 7]
    assert ngram.NgramIndex(tokens).propose(tokens, 5) == [2, 4, 7]


@pytest.mark.parametrize("max_n", [1, 2, 3, 4, 8])
def test_dict_equals_closed_form_random(max_n: int) -> None:
    rng = np.random.default_rng(max_n)
    for trial in range(400):
        length = int(rng.integers(0, 60))
        vocab = int(rng.integers(2, 6))  # tiny vocabulary: many overlapping matches
        tokens = rng.integers(0, vocab, size=length).tolist()
        k = int(rng.integers(0, 6))
        want = ngram.NgramIndex(tokens, max_n).propose(tokens, k)
        assert ngram.propose_closed_form(tokens, k, max_n) == want, (trial, tokens, k)


def test_dict_equals_closed_form_on_prefix_index() -> None:
    rng = np.random.default_rng(11)
    for _ in range(300):
        length = int(rng.integers(1, 50))
        tokens = rng.integers(0, 4, size=length).tolist()
        prefix = int(rng.integers(0, length + 1))
        want = ngram.NgramIndex(tokens[:prefix]).propose(tokens, 4)
        assert ngram.propose_closed_form(tokens, 4, index_len=prefix) == want


def test_dict_equals_closed_form_on_workload_histories() -> None:
    histories = workloads.drafting_histories(seed=3, batch=6, length=512)
    for max_n in (3, 4):
        for h in histories:
            tokens = h.tolist()
            assert ngram.propose_closed_form(tokens, 3, max_n) == ngram.NgramIndex(tokens, max_n).propose(tokens, 3)


def test_workload_histories_have_required_shape() -> None:
    histories = workloads.drafting_histories(seed=0)
    draft, lens = ngram.propose_batch([h.tolist() for h in histories], 3, max_n=3)
    assert histories.shape == (4, 512) and histories.dtype == np.int32
    assert lens[0] == 3  # repetitive tail: a full draft
    assert lens[-1] == 0  # the all-distinct history matches nothing
