"""CPU oracle for the verify step -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of each function on
the speculative-decoding verify path of NickWilde18/oxr-inference.  It is the
checker the GPU results are compared against, and the CPU baseline that
``bench.py`` times beside the GPU.  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s CPU-baseline leg may import it; the product package never
does, and has no CPU fallback.

Modules and the reference code each follows:

- ``bf16``       bfloat16 round-to-nearest-even helpers (torch CPU convention).
- ``ngram``      speculative.py:12-48 (``NgramProposer``, ``accept``), as the
                 reference's dict and as the closed form "largest (m(p), p)".
- ``norm_rope``  kernels.py:133-165 (``qk_norm_rope_store_reference``,
                 ``_sum_squares_reference``).
- ``attention``  attention.py:96-109 with the math of the reference test stub
                 (tests/test_language_fused.py:19-57).
- ``lm_head``    language.py:213-214 + decode_graph.py:167 (logits, first-index
                 argmax over bf16 logits) and engine.py:729-737 (accept and
                 length rollback).
- ``decoder``    language.py:69-104, 149-214, 247-317 (the verify forward
                 ``LanguageModel.extend`` of a Qwen3-style decoder).

How each function is pinned (golden vectors, known answers, invariants) is
listed in the test files under ``tests/`` that exercise it.
"""
