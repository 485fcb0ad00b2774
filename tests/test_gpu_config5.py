"""Configuration 5 at full size on gfx950 against the CPU oracle: the model bench.py times.

The synthetic Qwen-style decoder ``language.QWEN_SYNTHETIC`` (28 layers, hidden 2048, 16/8 heads,
head_dim 128, SwiGLU 6144, vocab 151,936, bf16, random init), block size 16.

- Teacher-forced layers 0, 13 and 27 at B=8, context 4096 (+4 new tokens), pages drawn from a
  65,536-page pool: the layer's output residual and the K/V rows it stores against the oracle's
  same layer from the same input, and pages the batch does not own left untouched.
- The device-resident :class:`VerifyLoop` (drafting, 28-layer forward, LM head + argmax,
  acceptance, rollback in one graph) at B = 1, 4, 8, 16 and contexts 4k, 16k and uniform
  1k-16k (B = 4 and 8; at B = 8 the attention runs on a per-step piece plan), two replays each
  against ``oracle.decoder.verify_step`` from the same state:
  * drafts bit-exact;
  * the step's LM head: its bf16 logits within one bf16 rounding of the exact product of the
    step's own final hidden states with the weight, and its greedy ids exactly the argmax of
    those logits;
  * the 28-layer forward as close to exact arithmetic as the oracle is: both are compared with
    the same forward computed without intermediate rounding (tests/unrounded_decoder.py), and
    the GPU's logit error may be at most 1.25x the oracle's.  Each layer's bf16 roundings (one
    ulp flips, 0.3% relative per layer in the teacher-forced check) compound over 28 layers, so
    both sit a few hundredths from exact logits;
  * greedy ids equal to the oracle's wherever the oracle's top-2 margin exceeds 10x the oracle's
    own RMS logit error (where it does not, the comparison continues from the GPU's ids);
  * accepted lengths, committed ids, KV lengths and histories equal to the oracle's acceptance of
    those ids.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import unrounded_decoder as unrounded
from conftest import announce, pkg
from oracle import decoder as oracle_decoder

pytestmark = pytest.mark.gpu
language = pkg("language")
kv_cache = pkg("kv_cache")
decode_graph = pkg("decode_graph")
lm_head = pkg("lm_head")
workloads = pkg("workloads")

CONFIG = language.QWEN_SYNTHETIC
BS = 16
ATOL, RTOL = 2e-2, 1e-2
# The GPU forward's RMS logit error against unrounded arithmetic, relative to the oracle's.
ERROR_RATIO = 1.25
# Ids must agree where the oracle's top-2 margin exceeds this many times its RMS logit error.
MARGIN_FACTOR = 10.0


@pytest.fixture(scope="module")
def model():
    announce("config 5 model (28 layers, vocab 151936)")
    weights = language.random_weights(CONFIG, 17_000, seed=0, device="cuda")
    cpu = weights.to("cpu")
    m = language.LanguageModel(CONFIG, weights)  # packs the GEMM weights
    del weights
    torch.cuda.synchronize()
    return m, cpu


class _LayerCaches:
    """The cache interface the forward reads (``k[layer]``, ``v[layer]``, ``block_size``) holding
    only the layers under test, each a full 65,536-page pool."""

    def __init__(self, layers, num_blocks: int, seed: int):
        g = torch.Generator(device="cuda").manual_seed(seed)
        shape = (num_blocks, BS, CONFIG.num_kv_heads, CONFIG.head_dim)
        self.k = {i: torch.randn(shape, generator=g, device="cuda").to(torch.bfloat16) for i in layers}
        self.v = {i: torch.randn(shape, generator=g, device="cuda").to(torch.bfloat16) for i in layers}
        self.block_size = BS


def _one_layer(cpu_w, layer: int, rows: torch.Tensor):
    """Oracle weights running one layer on ``rows`` (fed through the embedding as ids 0..t-1)."""
    from types import SimpleNamespace

    cfg = language.LanguageConfig(**{**CONFIG.__dict__, "num_layers": 1})
    w = SimpleNamespace(embed=rows, layers=[cpu_w.layers[layer]], final_norm=cpu_w.final_norm,
                        lm_head=cpu_w.lm_head, rope_cos=cpu_w.rope_cos, rope_sin=cpu_w.rope_sin)
    return cfg, w


def _rel_rms(got: torch.Tensor, want: torch.Tensor) -> float:
    got, want = got.float().cpu(), want.float().cpu()
    return ((got - want).pow(2).sum() / want.pow(2).sum()).sqrt().item()


@pytest.mark.parametrize("layer", [0, 13, 27])
def test_teacher_forced_layer(model, layer) -> None:
    m, cpu_w = model
    B, S, pool = 8, 4, 65_536
    rng = np.random.default_rng(100 + layer)
    pb = workloads.paged_batch(rng, B, S, (4100, 4100), block_size=BS, num_blocks=pool)
    caches = _LayerCaches([layer], pool, seed=200 + layer)
    t = B * S
    x = (torch.randn(t, CONFIG.hidden_size, generator=torch.Generator().manual_seed(layer)) * 0.5).to(torch.bfloat16)
    d = lambda a, dt: torch.from_numpy(np.asarray(a)).to(dt).cuda()
    eb = language.ExtendBatch(None, d(pb.positions, torch.int64), d(pb.slots, torch.int64),
                              d(pb.seq_lens, torch.int32), d(pb.block_table, torch.int32), S, ids=d(np.arange(t), torch.int64))
    # The oracle gets only the pages the batch uses, renumbered.
    used = np.unique(pb.block_table)
    remap = np.zeros(pool, dtype=np.int64)
    remap[used] = np.arange(len(used))
    idx = torch.from_numpy(used.astype(np.int64)).cuda()
    ck = caches.k[layer][idx].cpu()[None]
    cv = caches.v[layer][idx].cpu()[None]
    slots_c = remap[pb.slots // BS] * BS + pb.slots % BS
    table_c = remap[pb.block_table].astype(np.int32)

    spare = torch.from_numpy(np.setdiff1d(np.arange(pool), used)[:256].astype(np.int64)).cuda()
    spare_k, spare_v = caches.k[layer][spare].clone(), caches.v[layer][spare].clone()
    buffers = language.StepBuffers.allocate(CONFIG, B, S, pb.block_table.shape[1] * BS, "cuda")
    buffers.residual[:t].copy_(x.cuda())
    buffers.pending_splits = 0
    announce("teacher-forced layer", layer)
    m.run_layers(eb, caches, buffers, layer, layer + 1)
    m.settle(eb, buffers, cpu_w.final_norm.cuda())  # adds the layer's pending down_proj partials
    torch.cuda.synchronize()

    cfg, w = _one_layer(cpu_w, layer, x)
    trace = []
    oracle_decoder.extend(cfg, w, torch.arange(t), torch.from_numpy(pb.positions), torch.from_numpy(slots_c),
                          torch.from_numpy(pb.seq_lens), torch.from_numpy(table_c), S, ck, cv, trace=trace)
    rel = _rel_rms(buffers.residual[:t], trace[1])
    err = (buffers.residual[:t].float().cpu() - trace[1].float()).abs().max().item()
    print(f"layer {layer}: residual rel RMS {rel:.2e}, max abs {err:.3g}")
    assert rel < 1.5e-2 and err < 0.25, (rel, err)
    flat = lambda c: c.view(-1, CONFIG.num_kv_heads, CONFIG.head_dim)
    for got_cache, want_cache in ((caches.k[layer], ck[0]), (caches.v[layer], cv[0])):
        got = flat(got_cache)[torch.from_numpy(pb.slots).cuda()].float().cpu()
        want = flat(want_cache)[torch.from_numpy(slots_c)].float()
        assert bool(((got - want).abs() <= ATOL + RTOL * want.abs()).all()), (got - want).abs().max().item()
    # Pages the batch does not own keep their contents.
    for got_cache, before in ((caches.k[layer], spare_k), (caches.v[layer], spare_v)):
        assert torch.equal(got_cache[spare], before)


def _margins(logits: torch.Tensor) -> np.ndarray:
    values = logits.float().numpy()
    part = np.partition(values, -2, axis=-1)
    return part[:, -1] - part[:, -2]


# Per sequence and per row, the GPU's logit error against unrounded arithmetic relative to the
# oracle's for the same sequence / row.  The global ratio above averages over every row; these
# catch an error confined to one sequence (a lost context piece gives O(0.1-1) logit errors, ten
# or more times the oracle's 0.04) or to one row.  A row's error is a sum of many independent
# roundings, so its ratio scatters more than the sequence's.
SEQ_ERROR_RATIO = 1.6
ROW_ERROR_RATIO = 2.5


def _local_errors(err_gpu: torch.Tensor, err_ref: torch.Tensor, rows_per_seq: int) -> tuple[float, float]:
    """Worst per-sequence and per-row ratios of the GPU's RMS logit error to the oracle's."""
    row_g = err_gpu.pow(2).mean(-1).sqrt()
    row_r = err_ref.pow(2).mean(-1).sqrt()
    seq_g = err_gpu.view(-1, rows_per_seq * err_gpu.shape[-1]).pow(2).mean(-1).sqrt()
    seq_r = err_ref.view(-1, rows_per_seq * err_ref.shape[-1]).pow(2).mean(-1).sqrt()
    return (seq_g / seq_r).max().item(), (row_g / row_r).max().item()


def _loop_case(m, B: int, ctx: tuple[int, int], seed: int, steps: int):
    rng = np.random.default_rng(seed)
    k, S = 3, 4
    seq_lens = rng.integers(ctx[0], ctx[1] + 1, size=B).astype(np.int32)
    width = -(-(int(seq_lens.max()) + S * (steps + 2) + S) // BS)
    num_blocks = B * width + 16
    cache = kv_cache.KVCache(CONFIG.num_layers, CONFIG.num_kv_heads, CONFIG.head_dim, num_blocks, block_size=BS)
    g = torch.Generator(device="cuda").manual_seed(seed)
    for layer in range(CONFIG.num_layers):
        cache.k[layer].normal_(generator=g)
        cache.v[layer].normal_(generator=g)
    table = rng.permutation(num_blocks)[: B * width].astype(np.int32).reshape(B, width)
    histories = [workloads.repetitive_history(rng, 1024, repetitive_tail=True) for _ in range(B)]
    loop = decode_graph.VerifyLoop(m, cache, batch=B, k=k, max_n=4, history_capacity=1024 + S * (steps + 4),
                                   table_width=width)
    loop.load(histories, seq_lens, table)
    return loop, cache, table, histories, seq_lens


def _exact_head_check(hidden: torch.Tensor, weight: torch.Tensor, got_logits: torch.Tensor) -> None:
    """The LM head of the step: bf16 logits within one bf16 rounding (plus fp32 accumulation-order
    slack) of the exact product hidden @ weight^T, computed in float64 from the same bf16 inputs."""
    h = hidden.double()
    worst = 0.0
    for r in range(0, weight.shape[0], 16384):
        exact = h @ weight[r : r + 16384].double().T
        got = got_logits[:, r : r + 16384].double()
        # One bf16 rounding is at most half an ulp: 2^-9 relative; fp32 accumulation adds ~1e-6.
        bound = exact.abs() * 2.0 ** -8 + 1e-5
        over = ((got - exact).abs() - bound).max().item()
        worst = max(worst, over)
    assert worst <= 0.0, worst


@pytest.mark.parametrize("B,ctx", [(8, (4096, 4096)), (1, (4096, 4096)), (16, (4096, 4096)), (1, (16384, 16384)),
                                   (4, (1024, 16384)), (8, (1024, 16384))])
def test_verify_loop_full_size(model, B, ctx) -> None:
    m, cpu_w = model
    steps = 2
    loop, cache, table, histories, seq_lens = _loop_case(m, B, ctx, seed=300 + B + ctx[0], steps=steps)
    S, k = loop.tokens_per_seq, loop.k
    # Mixed contexts at B >= 8 (here 4.3x apart) run the attention on a per-step piece plan.
    assert loop.buffers.balanced == (ctx[0] != ctx[1] and B >= decode_graph.BALANCE_MIN_BATCH)
    announce("config 5 verify loop", B, ctx, "planned" if loop.buffers.balanced else "even")
    loop.capture()
    hist = [list(map(int, h)) for h in histories]
    lens = [int(x) for x in seq_lens]
    for step in range(steps):
        cpu_k, cpu_v = cache.k.cpu(), cache.v.cpu()
        announce("config 5 step", B, ctx, step)
        loop.replay()
        got_pred = loop.buffers.predicted[: B * S].cpu().numpy()
        got_hidden = loop.buffers.h[: B * S].cpu()
        got_logits = lm_head.logits(loop.buffers.h[: B * S], m.weights.lm_head).cpu()
        torch.cuda.synchronize()
        want = oracle_decoder.verify_step(CONFIG, cpu_w, hist, np.array(lens), table, k, 4, cpu_k, cpu_v, BS,
                                          max_positions=loop.max_positions)
        got_draft = loop.inputs.draft.cpu().numpy()
        got_len = loop.inputs.draft_len.cpu().numpy()
        assert [got_draft[b, : got_len[b]].tolist() for b in range(B)] == want.drafts

        # The step's LM head and argmax, exactly.
        _exact_head_check(got_hidden, cpu_w.lm_head, got_logits)
        assert np.array_equal(got_pred, got_logits.float().argmax(-1).numpy())

        # The forward: no further from unrounded arithmetic than the oracle.
        ids, positions, _, attn_lens = oracle_decoder.verify_rows(hist, want.drafts, lens, table, S, BS)
        _, exact = unrounded.extend(CONFIG, cpu_w, ids, positions, attn_lens, table, S, cpu_k, cpu_v, BS,
                                    dtype=torch.float32, with_logits=True)
        rms = lambda e: e.pow(2).mean().sqrt().item()
        err_gpu = got_logits.float() - exact
        err_ref = want.logits.float() - exact
        margin = _margins(want.logits)
        want_pred = want.predicted.reshape(-1).numpy()
        clear = margin > MARGIN_FACTOR * rms(err_ref)
        differ = np.flatnonzero(got_pred != want_pred)
        print(f"B={B} ctx={ctx} step {step}: logit RMS error vs unrounded: gpu {rms(err_gpu):.4f}, oracle "
              f"{rms(err_ref):.4f}; gpu-oracle max {(got_logits.float() - want.logits.float()).abs().max().item():.3f}; "
              f"clear rows {clear.mean():.2f}; ids differ at {differ.tolist()} (margins {margin[differ].round(3).tolist()})")
        seq_ratio, row_ratio = _local_errors(err_gpu, err_ref, S)
        print(f"  worst per-sequence error ratio {seq_ratio:.3f}, per-row {row_ratio:.3f}")
        assert rms(err_gpu) <= ERROR_RATIO * rms(err_ref)
        assert seq_ratio <= SEQ_ERROR_RATIO and row_ratio <= ROW_ERROR_RATIO
        assert np.array_equal(got_pred[clear], want_pred[clear])

        taken, new_lens = oracle_decoder.accept_step(want.drafts, got_pred.reshape(B, S), lens)
        assert loop.accepted.accepted.cpu().numpy().tolist() == [len(t) - 1 for t in taken]
        committed = loop.accepted.committed.cpu().numpy()
        assert [committed[b, : len(taken[b])].tolist() for b in range(B)] == taken
        assert loop.seq_len.cpu().numpy().tolist() == new_lens
        hl = loop.history_len.cpu().numpy()
        hist = [h + t for h, t in zip(hist, taken)]
        assert [loop.history[b, : hl[b]].cpu().tolist() for b in range(B)] == hist
        lens = new_lens
    del loop, cache
    torch.cuda.empty_cache()


def test_decode_graphs_full_size(model) -> None:
    """``DecodeGraphs`` (decode_graph.py:33-119) at the benchmark's shape: the 28-layer model, 8
    sequences with one new token each after 4096 context keys, pages from a permuted pool.  Logits
    and greedy ids against ``oracle.decoder.extend`` with one token per sequence, under the verify
    loop's criterion: RMS logit error against unrounded arithmetic at most ERROR_RATIO x the
    oracle's (and per sequence / per row as above); ids equal wherever the oracle's top-2 margin
    exceeds MARGIN_FACTOR x its RMS error; and the graph's ids are exactly the argmax of its logits."""
    m, cpu_w = model
    B, ctx = 8, 4096
    rng = np.random.default_rng(777)
    width = -(-(ctx + 1) // BS) + 1
    num_blocks = B * width + 16
    cache = kv_cache.KVCache(CONFIG.num_layers, CONFIG.num_kv_heads, CONFIG.head_dim, num_blocks, block_size=BS)
    g = torch.Generator(device="cuda").manual_seed(777)
    for layer in range(CONFIG.num_layers):
        cache.k[layer].normal_(generator=g)
        cache.v[layer].normal_(generator=g)
    announce("config 5 decode graphs", B, ctx)
    graphs = decode_graph.DecodeGraphs(m, cache, max_batch=B, max_positions=width * BS)
    pages = [p for p in rng.permutation(num_blocks).tolist() if p != graphs.scratch_block]
    tables = [pages[width * b : width * (b + 1)] for b in range(B)]
    ids = rng.integers(0, CONFIG.vocab_size, size=B).tolist()
    positions = [ctx] * B
    slots = [tables[b][ctx // BS] * BS + ctx % BS for b in range(B)]
    seq_lens = [ctx + 1] * B
    cpu_k, cpu_v = cache.k.cpu(), cache.v.cpu()
    logits, tokens = graphs.run(ids, positions, slots, seq_lens, tables)
    got_logits, got_ids = logits.cpu(), tokens.cpu().numpy()
    torch.cuda.synchronize()
    assert np.array_equal(got_ids, got_logits.float().argmax(-1).numpy())
    table = torch.tensor(tables, dtype=torch.int32)
    announce("config 5 decode graphs: oracle")
    want_hidden = oracle_decoder.extend(CONFIG, cpu_w, torch.tensor(ids), torch.tensor(positions), torch.tensor(slots),
                                        torch.tensor(seq_lens, dtype=torch.int32), table, 1, cpu_k.clone(),
                                        cpu_v.clone())
    want_logits = oracle_decoder.logits(cpu_w, want_hidden)
    _, exact = unrounded.extend(CONFIG, cpu_w, ids, positions, seq_lens, table.numpy(), 1, cpu_k, cpu_v, BS,
                                dtype=torch.float32, with_logits=True)
    rms = lambda e: e.pow(2).mean().sqrt().item()
    err_gpu = got_logits.float() - exact
    err_ref = want_logits.float() - exact
    margin = _margins(want_logits)
    want_ids = want_logits.float().argmax(-1).numpy()
    clear = margin > MARGIN_FACTOR * rms(err_ref)
    seq_ratio, row_ratio = _local_errors(err_gpu, err_ref, 1)
    print(f"decode B={B} ctx={ctx}: logit RMS error vs unrounded: gpu {rms(err_gpu):.4f}, oracle {rms(err_ref):.4f}; "
          f"worst row ratio {row_ratio:.3f}; clear rows {clear.mean():.2f}; ids differ at "
          f"{np.flatnonzero(got_ids != want_ids).tolist()}")
    assert rms(err_gpu) <= ERROR_RATIO * rms(err_ref)
    assert row_ratio <= ROW_ERROR_RATIO
    assert np.array_equal(got_ids[clear], want_ids[clear])
    del graphs, cache
    torch.cuda.empty_cache()

