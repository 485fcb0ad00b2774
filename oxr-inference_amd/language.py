"""Qwen3-style decoder verify forward on gfx950 kernels: the drop-in for the verify half of
oxr_runtime/language.py (``LanguageModel.extend`` + ``logits``, language.py:149-214, 247-317).

Per layer (language.py:301-317 with the fused projections of :234-245):

    h        = rms_norm(residual)                               oxr_rms_norm / oxr_embed_rms_norm
    qkv      = h @ Wqkv^T                                       oxr_gemm_bf16
    q        = qk_norm_rope_store(qkv, ...)  (K/V -> cache)     } one launch:
    attn     = paged_extend(q, cache, seq_lens, block_table)    } oxr_qk_norm_rope_paged_extend
    o_part   = k-split fp32 sums of attn @ Wo^T                 oxr_gemm_bf16_partial
    residual = bf16(bf16(sum o_part) + residual); h = rms_norm  oxr_add_partials_rms_norm
    act      = silu(h @ Wg^T) * (h @ Wu^T)                      oxr_gemm_bf16 (SiLU*mul epilogue)
    d_part   = k-split fp32 sums of act @ Wd^T                  oxr_gemm_bf16_partial

and the next layer's input norm (or the final norm) starts with the residual add of d_part.
o_proj and down_proj have only 2048 output columns: split over k so every CU streams weights,
their partials are summed by the norm that follows, which also does ``_add_rms_norm``'s residual
add (language.py:94-99) with the reference's rounding points (GEMM output rounded to bf16, then
added, residual stored in bf16 before it is normalised).

All intermediate buffers live in a preallocated :class:`StepBuffers`, so a forward enqueues
kernels only and can be captured in a HIP graph.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _lib, attention, gemm, lm_head, mlp
from .gemm import Weight
from .kv_cache import KVCache


@dataclass(frozen=True)
class LanguageConfig:
    """The shapes language.py reads from config.json (config.py:38-50)."""

    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    rms_norm_eps: float
    rope_theta: float
    vocab_size: int

    @property
    def qkv_size(self) -> int:
        return (self.num_heads + 2 * self.num_kv_heads) * self.head_dim


# The synthetic Qwen-style decoder of the verify benchmark (28 layers, hidden 2048, 16/8 heads).
QWEN_SYNTHETIC = LanguageConfig(2048, 6144, 28, 16, 8, 128, 1e-6, 1e6, 151_936)


_MATRICES = ("qkv", "o", "gate_up", "down")


@dataclass
class LayerWeights:
    input_norm: torch.Tensor   # [hidden]
    qkv: Weight                # [(H + 2KV) * D, hidden]  (q | k | v rows, language.py:237)
    q_norm: torch.Tensor       # [D]
    k_norm: torch.Tensor       # [D]
    o: Weight                  # [hidden, H * D]
    post_norm: torch.Tensor    # [hidden]
    gate_up: Weight            # [2 * intermediate, hidden]  (gate rows then up rows, language.py:238)
    down: Weight               # [hidden, intermediate]

    def _map(self, matrix) -> "LayerWeights":
        return LayerWeights(**{f: matrix(getattr(self, f)) if f in _MATRICES else getattr(self, f)
                               for f in LayerWeights.__dataclass_fields__})


@dataclass
class LanguageWeights:
    """The decoder's weights.  GEMM matrices (the four per layer and the LM head) are row-major
    ``torch.Tensor``s as a checkpoint holds them, or :class:`~.gemm.PackedWeight`s after
    :meth:`packed` -- the form :class:`LanguageModel` runs on."""

    embed: torch.Tensor        # [vocab, hidden]
    layers: list[LayerWeights]
    final_norm: torch.Tensor   # [hidden]
    lm_head: Weight            # [vocab, hidden]
    rope_cos: torch.Tensor     # [max_positions, D/2] bf16
    rope_sin: torch.Tensor

    def to(self, device) -> "LanguageWeights":
        mv = lambda t: t.to(device)
        return LanguageWeights(
            mv(self.embed), [LayerWeights(*(mv(getattr(l, f)) for f in LayerWeights.__dataclass_fields__)) for l in self.layers],
            mv(self.final_norm), mv(self.lm_head), mv(self.rope_cos), mv(self.rope_sin),
        )

    def _map_matrices(self, matrix) -> "LanguageWeights":
        return LanguageWeights(self.embed, [l._map(matrix) for l in self.layers], self.final_norm, matrix(self.lm_head),
                               self.rope_cos, self.rope_sin)

    def packed(self) -> "LanguageWeights":
        """Every GEMM matrix packed once on its GPU (``gemm.pack_weight``); other tensors shared."""
        return self._map_matrices(lambda w: w if isinstance(w, gemm.PackedWeight) else gemm.pack_weight(w))

    def unpacked(self) -> "LanguageWeights":
        """Every GEMM matrix row-major again; other tensors shared."""
        return self._map_matrices(lambda w: w.unpack() if isinstance(w, gemm.PackedWeight) else w)

    @classmethod
    def from_state_dict(cls, config: LanguageConfig, state: dict[str, torch.Tensor], max_positions: int, *,
                        device=None, dtype: torch.dtype = torch.bfloat16) -> "LanguageWeights":
        """The reference ``LanguageModel``'s parameters by name (language.py:155-158, 221-231):
        ``embed_tokens``, ``layers.{i}.{input_layernorm, q_proj, k_proj, v_proj, o_proj, q_norm,
        k_norm, post_attention_layernorm, gate_proj, up_proj, down_proj}``, ``norm``, ``lm_head``
        (each ``.weight``); after the reference's ``fuse_projections`` (language.py:234-245)
        ``qkv_proj`` / ``gate_up_proj`` instead of the split ones.  q/k/v and gate/up are
        concatenated in that order, as ``fuse_projections`` does.  Every name must be used exactly
        once and every shape must match, else ``KeyError`` / ``ValueError`` (the reference loader's
        rules, weights.py:17-44).  The RoPE tables are computed (the reference's are non-persistent
        buffers, language.py:160-165)."""
        c = config
        used: set[str] = set()

        def take(name: str, shape: tuple[int, ...]) -> torch.Tensor:
            if name not in state:
                raise KeyError(f"missing parameter {name}")
            t = state[name]
            if tuple(t.shape) != shape:
                raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {shape}")
            used.add(name)
            return t.to(device=device if device is not None else t.device, dtype=dtype).contiguous()

        def fused(prefix: str, fused_name: str, parts: list[tuple[str, int]], cols: int) -> torch.Tensor:
            rows = sum(n for _, n in parts)
            if f"{prefix}{fused_name}.weight" in state:
                return take(f"{prefix}{fused_name}.weight", (rows, cols))
            return torch.cat([take(f"{prefix}{name}.weight", (n, cols)) for name, n in parts])

        h, d = c.hidden_size, c.head_dim
        layers = []
        for i in range(c.num_layers):
            p = f"layers.{i}."
            layers.append(LayerWeights(
                take(p + "input_layernorm.weight", (h,)),
                fused(p, "qkv_proj", [("q_proj", c.num_heads * d), ("k_proj", c.num_kv_heads * d),
                                      ("v_proj", c.num_kv_heads * d)], h),
                take(p + "q_norm.weight", (d,)), take(p + "k_norm.weight", (d,)),
                take(p + "o_proj.weight", (h, c.num_heads * d)),
                take(p + "post_attention_layernorm.weight", (h,)),
                fused(p, "gate_up_proj", [("gate_proj", c.intermediate_size), ("up_proj", c.intermediate_size)], h),
                take(p + "down_proj.weight", (h, c.intermediate_size)),
            ))
        embed = take("embed_tokens.weight", (c.vocab_size, h))
        final_norm = take("norm.weight", (h,))
        head = take("lm_head.weight", (c.vocab_size, h))
        unused = sorted(set(state) - used - {"rope_cos", "rope_sin"})
        if unused:
            raise KeyError(f"parameters with no place in the model: {unused[:8]}{' ...' if len(unused) > 8 else ''}")
        cos, sin = rope_tables(c, max_positions)
        return cls(embed, layers, final_norm, head, cos.to(embed.device), sin.to(embed.device))


def rope_tables(config: LanguageConfig, max_positions: int) -> tuple[torch.Tensor, torch.Tensor]:
    """language.py:160-170: fp32 angles ``position * theta^(-2i/D)``, cos/sin, stored as bf16."""
    inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, config.head_dim, 2, dtype=torch.float) / config.head_dim))
    freqs = torch.outer(torch.arange(max_positions, dtype=torch.float), inv_freq)
    return freqs.cos().to(torch.bfloat16), freqs.sin().to(torch.bfloat16)


def random_weights(config: LanguageConfig, max_positions: int, *, seed: int = 0, device="cuda",
                   std: float = 0.02) -> LanguageWeights:
    """Random-init weights (no checkpoint): matrices ~N(0, std), norm weights ~U(0.5, 1.5)."""
    g = torch.Generator(device=device).manual_seed(seed)
    c = config

    def mat(*shape):
        return (torch.randn(*shape, generator=g, device=device) * std).to(torch.bfloat16)

    def norm(n):
        return (0.5 + torch.rand(n, generator=g, device=device)).to(torch.bfloat16)

    layers = [
        LayerWeights(
            norm(c.hidden_size), mat(c.qkv_size, c.hidden_size), norm(c.head_dim), norm(c.head_dim),
            mat(c.hidden_size, c.num_heads * c.head_dim), norm(c.hidden_size),
            mat(2 * c.intermediate_size, c.hidden_size), mat(c.hidden_size, c.intermediate_size),
        )
        for _ in range(c.num_layers)
    ]
    cos, sin = rope_tables(c, max_positions)
    return LanguageWeights(mat(c.vocab_size, c.hidden_size), layers, norm(c.hidden_size),
                           mat(c.vocab_size, c.hidden_size), cos.to(device), sin.to(device))


def _check_batch_inputs(embeds: torch.Tensor | None, ids: torch.Tensor | None, what: str) -> None:
    """Exactly one of ``embeds`` (bf16 rows, the reference's field) and ``ids`` (int64 token ids)."""
    if (embeds is None) == (ids is None):
        raise ValueError(f"{what}: give either embeds (bf16 [T, hidden]) or ids= (int64 [T]), not both or neither")
    if ids is not None and ids.dtype != torch.int64:
        raise TypeError(f"{what}: ids must be int64 token ids, got {ids.dtype}")
    if embeds is not None and embeds.dtype != torch.bfloat16:
        hint = " (token ids go in ids=)" if not embeds.is_floating_point() else ""
        raise TypeError(f"{what}: embeds must be bf16 [T, hidden], got {embeds.dtype}{hint}")


@dataclass
class ExtendBatch:
    """One verify step: every sequence brings the same number S of new tokens (language.py:122-136).

    The fields keep the reference's order, so the reference's callers build it unchanged:
    ``ExtendBatch(embed_tokens(ids), positions, slots, seq_lens, block_table, S)`` (engine.py:716-724,
    decode_graph.py:163-166).  This build's own callers pass ``embeds=None`` and the token ids as
    ``ids=``: the embedding gather then runs inside layer 0's input norm (one launch fewer)."""

    embeds: torch.Tensor | None  # bf16 [B * S, hidden]
    positions: torch.Tensor   # int64 [B * S]
    slots: torch.Tensor       # int64 [B * S]
    seq_lens: torch.Tensor    # int32 [B], including the S new tokens
    block_table: torch.Tensor  # int32 [B, max_blocks]
    tokens_per_seq: int
    ids: torch.Tensor | None = None  # int64 [B * S], in place of embeds

    def __post_init__(self) -> None:
        _check_batch_inputs(self.embeds, self.ids, "ExtendBatch")


@dataclass
class DecodeBatch:
    """One decode step: one new token per sequence (language.py:54-66), fields in the reference's order
    (``DecodeBatch(embed_tokens(ids), positions, slots, seq_lens, block_table)``, engine.py:594-600);
    as with :class:`ExtendBatch`, ``ids=`` may replace ``embeds``."""

    embeds: torch.Tensor | None  # bf16 [B, hidden]
    positions: torch.Tensor   # int64 [B]
    slots: torch.Tensor       # int64 [B]
    seq_lens: torch.Tensor    # int32 [B], including the new token
    block_table: torch.Tensor  # int32 [B, max_blocks]
    ids: torch.Tensor | None = None  # int64 [B], in place of embeds

    def __post_init__(self) -> None:
        _check_batch_inputs(self.embeds, self.ids, "DecodeBatch")

    def as_extend(self) -> ExtendBatch:
        return ExtendBatch(self.embeds, self.positions, self.slots, self.seq_lens, self.block_table, 1, ids=self.ids)


@dataclass
class StepBuffers:
    """Every intermediate of one forward, allocated once for up to ``max_tokens`` rows."""

    residual: torch.Tensor
    h: torch.Tensor                 # row-major: the final norm's output (the LM head's input)
    h_packed: gemm.PackedMatrix     # the layers' norm outputs, packed x of qkv / gate_up
    qkv: torch.Tensor
    attn: gemm.PackedMatrix         # [B * S, H * D] packed x of o_proj
    act: gemm.PackedMatrix          # [B * S, intermediate] packed x of down_proj
    attn_workspace: torch.Tensor
    head_workspace: torch.Tensor
    predicted: torch.Tensor
    partials: torch.Tensor  # fp32 k-split sums of o_proj / down_proj, consumed by the next norm
    max_tokens: int
    max_seq_len: int
    max_batch: int = field(default=0)
    pending_splits: int = field(default=0)  # partials not yet added to the residual (0: none)
    # The one-launch MLP block (mlp.mlp_block, up to mlp.MAX_ROWS rows): its 8 output slices, the
    # residual it writes (the next norm reads it there and stores the sum to `residual`), workspace.
    mlp_partials: torch.Tensor | None = field(default=None)
    residual_alt: torch.Tensor | None = field(default=None)
    mlp_workspace: torch.Tensor | None = field(default=None)
    pending_partials: torch.Tensor | None = field(default=None)  # the pending splits' buffer (None: partials)
    pending_from_alt: bool = field(default=False)  # the pending residual is in residual_alt
    # Context-piece plan of the attention launches (attention.build_plan), rebuilt from the step's
    # seq_lens at the start of run_layers when `balanced` is set (contexts of different lengths).
    attn_plan: torch.Tensor | None = field(default=None)
    balanced: bool = field(default=False)

    @classmethod
    def allocate(cls, config: LanguageConfig, max_batch: int, tokens_per_seq: int, max_seq_len: int,
                 device) -> "StepBuffers":
        t = max_batch * tokens_per_seq
        bf = dict(dtype=torch.bfloat16, device=device)
        return cls(
            residual=torch.zeros(t, config.hidden_size, **bf), h=torch.zeros(t, config.hidden_size, **bf),
            h_packed=gemm.packed_rows(t, config.hidden_size, device),
            qkv=torch.zeros(t, config.qkv_size, **bf),
            attn=gemm.packed_rows(t, config.num_heads * config.head_dim, device),
            act=gemm.packed_rows(t, config.intermediate_size, device),
            attn_workspace=torch.zeros(max(attention.workspace_bytes(max_batch, config.num_kv_heads, max_seq_len), 1),
                                       dtype=torch.uint8, device=device),
            head_workspace=torch.zeros(max(lm_head.workspace_bytes(t, config.vocab_size), 1), dtype=torch.uint8,
                                       device=device),
            predicted=torch.zeros(t, dtype=torch.int64, device=device),
            partials=torch.zeros(max(gemm.partial_splits(config.hidden_size, config.num_heads * config.head_dim),
                                     gemm.partial_splits(config.hidden_size, config.intermediate_size)),
                                 t, config.hidden_size, dtype=torch.float32, device=device),
            max_tokens=t, max_seq_len=max_seq_len, max_batch=max_batch,
            mlp_partials=(torch.zeros(mlp.SPLITS_OUT, t, config.hidden_size, dtype=torch.float32, device=device)
                          if t <= mlp.MAX_ROWS else None),
            residual_alt=torch.zeros(t, config.hidden_size, **bf) if t <= mlp.MAX_ROWS else None,
            mlp_workspace=mlp.workspace(device) if t <= mlp.MAX_ROWS else None,
        )

    def enable_plan(self, config: LanguageConfig, tokens_per_seq: int) -> None:
        """Run the attention launches on a per-step context-piece plan from now on (allocates the plan's
        room once: call before any graph capture)."""
        if self.attn_plan is None:
            self.attn_plan = _plan_buffer(config, self.max_batch, tokens_per_seq, self.max_seq_len,
                                          self.residual.device)
        self.balanced = True


def _plan_buffer(config: LanguageConfig, max_batch: int, tokens_per_seq: int, max_seq_len: int,
                 device) -> torch.Tensor | None:
    """Room for the attention plan of any batch up to ``max_batch`` (None if none ever splits)."""
    n = max((attention.plan_ints(b, tokens_per_seq, config.num_heads, config.num_kv_heads, max_seq_len)
             for b in range(1, max_batch + 1)), default=0)
    return torch.zeros(n, dtype=torch.int32, device=device) if n else None


class LanguageModel:
    """Verify forward (``extend``) and LM head of the decoder on gfx950 kernels.

    The GEMM matrices are packed once here (``weights.packed()``, a copy: drop the row-major
    ``weights`` afterwards to free them); ``self.weights`` holds the packed set."""

    def __init__(self, config: LanguageConfig, weights: LanguageWeights):
        self.config = config
        self.weights = weights.packed()
        # gate_up with rows interleaved by 8, for the one-launch MLP block (mlp.mlp_block) where the
        # device and shape take it; None elsewhere (the three-launch form runs).
        self.mlp_gate_up: list[gemm.PackedMatrix] | None = None
        if config.num_layers and mlp.supported(1, config.hidden_size, config.intermediate_size):
            self.mlp_gate_up = [gemm.pack_weight(mlp.interleave_gate_up(layer.gate_up.unpack()))
                                for layer in self.weights.layers]

    def extend(self, batch: ExtendBatch, cache: KVCache, buffers: StepBuffers | None = None) -> torch.Tensor:
        """``[B * S, hidden]``: the final-norm hidden state of every new token (language.py:201-211).
        K/V of the new tokens are written into ``cache`` at ``batch.slots``."""
        buffers = self._buffers(batch, cache, buffers)
        self.embed(batch, buffers)
        self.run_layers(batch, cache, buffers, 0, self.config.num_layers, first_norm_done=True)
        return self.final_norm(batch, buffers)

    def decode(self, batch: DecodeBatch, cache: KVCache, buffers: StepBuffers | None = None) -> torch.Tensor:
        """``[B, hidden]``: the final-norm hidden state of each sequence's new token (language.py:190-199).
        The verify forward with one token per sequence: the same kernels, attention as
        ``paged_decode``."""
        return self.extend(batch.as_extend(), cache, buffers)

    def embed_tokens(self, ids: torch.Tensor) -> torch.Tensor:
        """The reference's ``embed_tokens`` module (an ``nn.Embedding``, language.py:155) as its eager
        decode and verify paths call it (engine.py:595, 717): bf16 ``[*ids.shape, hidden]``, the
        embedding table's rows of integer ``ids``.  Ids outside ``[0, vocab)`` are clamped (the
        reference's callers clamp negative ids themselves, model.py:32)."""
        if ids.dtype not in (torch.int64, torch.int32):
            raise TypeError(f"embed_tokens: ids must be int64 or int32, got {ids.dtype}")
        _lib.require_gpu(ids, name="embed_tokens")
        c, table = self.config, self.weights.embed
        flat = ids.reshape(-1).to(torch.int64).contiguous()
        out = torch.empty(flat.numel(), c.hidden_size, dtype=torch.bfloat16, device=ids.device)
        _lib.call("oxr_embed_gather", flat.data_ptr(), flat.numel(), table.data_ptr(), c.vocab_size, c.hidden_size,
                  out.data_ptr(), c.hidden_size, _lib.stream(ids.device))
        return out.view(*ids.shape, c.hidden_size)

    def _buffers(self, batch: ExtendBatch, cache: KVCache, buffers: StepBuffers | None) -> StepBuffers:
        _lib.require_gpu(batch.positions, batch.slots, batch.seq_lens, batch.block_table, name="extend")
        b, s = batch.block_table.shape[0], batch.tokens_per_seq
        if buffers is None:
            buffers = StepBuffers.allocate(self.config, b, s, batch.block_table.shape[1] * cache.block_size,
                                           batch.positions.device)
        _lib.require(b * s <= buffers.max_tokens and b <= buffers.max_batch, "extend: batch larger than the buffers")
        return buffers

    def embed(self, batch: ExtendBatch, buffers: StepBuffers) -> None:
        """residual = embed_tokens(ids) (decode_graph.py:164), or the caller's ``embeds``; h = layer 0's
        input norm of it."""
        buffers.pending_splits, buffers.pending_partials, buffers.pending_from_alt = 0, None, False
        c, w = self.config, self.weights
        t = batch.block_table.shape[0] * batch.tokens_per_seq
        res = buffers.residual[:t]
        stream = _lib.stream(batch.positions.device)
        if batch.ids is not None:
            _lib.call("oxr_embed_rms_norm", batch.ids.data_ptr(), t, w.embed.data_ptr(), c.vocab_size, c.hidden_size,
                      w.layers[0].input_norm.data_ptr(), float(c.rms_norm_eps), res.data_ptr(),
                      buffers.h_packed.data.data_ptr(), 1, stream)
        else:
            _lib.require(tuple(batch.embeds.shape) == (t, c.hidden_size),
                         f"extend: embeds has shape {tuple(batch.embeds.shape)}, expected {(t, c.hidden_size)}")
            res.copy_(batch.embeds)
            self._norm(res, w.layers[0].input_norm, buffers.h_packed.view_rows(t), stream)

    def _norm(self, x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | gemm.PackedMatrix, stream: int) -> None:
        c = self.config
        packed = isinstance(out, gemm.PackedMatrix)
        _lib.call("oxr_rms_norm", x.data_ptr(), x.stride(0), x.shape[0], c.hidden_size, weight.data_ptr(),
                  float(c.rms_norm_eps), out.data.data_ptr() if packed else out.data_ptr(),
                  0 if packed else out.stride(0), 1 if packed else 0, stream)

    def _settle_norm(self, buffers: StepBuffers, t: int, weight: torch.Tensor, stream: int, *,
                     packed: bool = True) -> None:
        """h = rms_norm(residual) * weight, first adding any pending GEMM partials to the residual;
        into ``buffers.h_packed`` (the next layer GEMM's x) or, with ``packed=False``, ``buffers.h``."""
        res = buffers.residual[:t]
        h = buffers.h_packed.view_rows(t) if packed else buffers.h[:t]
        if buffers.pending_splits:
            partials = buffers.partials if buffers.pending_partials is None else buffers.pending_partials
            gemm.add_partials_rms_norm(partials, buffers.pending_splits, res, weight, self.config.rms_norm_eps, h,
                                       residual_in=buffers.residual_alt[:t] if buffers.pending_from_alt else None)
            buffers.pending_splits, buffers.pending_partials, buffers.pending_from_alt = 0, None, False
        else:
            self._norm(res, weight, h, stream)

    def run_layers(self, batch: ExtendBatch, cache: KVCache, buffers: StepBuffers, start: int, stop: int, *,
                   first_norm_done: bool = False) -> None:
        """Layers ``[start, stop)`` on ``buffers.residual`` (the residual stream after the previous
        layer's MLP add).  The last layer's down_proj is left as pending partials: the next norm
        (``run_layers``, ``final_norm`` or ``settle``) adds it to the residual."""
        c, w = self.config, self.weights
        b, s = batch.block_table.shape[0], batch.tokens_per_seq
        t = b * s
        stream = _lib.stream(batch.positions.device)
        h = buffers.h_packed.view_rows(t)
        qkv = buffers.qkv[:t]
        attn, act = buffers.attn.view_rows(t), buffers.act.view_rows(t)
        max_seq_len = min(buffers.max_seq_len, batch.block_table.shape[1] * cache.block_size)
        eps = float(c.rms_norm_eps)
        plan = None
        if buffers.balanced and buffers.attn_plan is not None:
            plan = attention.build_plan(batch.seq_lens, s, c.num_heads, c.num_kv_heads, max_seq_len,
                                        out=buffers.attn_plan)
        use_mlp_block = (self.mlp_gate_up is not None and buffers.mlp_workspace is not None
                         and t <= mlp.MAX_ROWS)
        for index in range(start, stop):
            layer = w.layers[index]
            if not (first_norm_done and index == start):
                self._settle_norm(buffers, t, layer.input_norm, stream)
            gemm.linear(h, layer.qkv, out=qkv)
            k_cache, v_cache = cache.k[index], cache.v[index]
            attention.qk_norm_rope_paged_extend(
                qkv, layer.q_norm, layer.k_norm, w.rope_cos, w.rope_sin, batch.positions, eps, k_cache, v_cache,
                batch.slots, batch.seq_lens, batch.block_table, c.num_heads, scale=c.head_dim ** -0.5,
                max_seq_len=max_seq_len, out=attn, workspace=buffers.attn_workspace, plan=plan,
            )
            buffers.pending_splits = gemm.linear_partial(attn, layer.o, buffers.partials)
            buffers.pending_partials, buffers.pending_from_alt = None, False
            if use_mlp_block:
                mlp.mlp_block(buffers.partials, buffers.pending_splits, buffers.residual[:t], layer.post_norm, eps,
                              self.mlp_gate_up[index], layer.down, buffers.residual_alt[:t], buffers.mlp_partials,
                              buffers.mlp_workspace)
                buffers.pending_splits, buffers.pending_partials = mlp.SPLITS_OUT, buffers.mlp_partials
                buffers.pending_from_alt = True
                continue
            self._settle_norm(buffers, t, layer.post_norm, stream)
            gemm.linear_silu_mul(h, layer.gate_up, out=act)
            buffers.pending_splits = gemm.linear_partial(act, layer.down, buffers.partials)

    def settle(self, batch: ExtendBatch, buffers: StepBuffers, weight: torch.Tensor, *, packed: bool = True) -> None:
        """Add pending partials to the residual (and normalise it with ``weight`` into
        ``h_packed``, or ``h`` with ``packed=False``)."""
        t = batch.block_table.shape[0] * batch.tokens_per_seq
        self._settle_norm(buffers, t, weight, _lib.stream(batch.positions.device), packed=packed)

    def final_norm(self, batch: ExtendBatch, buffers: StepBuffers) -> torch.Tensor:
        t = batch.block_table.shape[0] * batch.tokens_per_seq
        self._settle_norm(buffers, t, self.weights.final_norm, _lib.stream(batch.positions.device), packed=False)
        return buffers.h[:t]

    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        """bf16 ``hidden @ lm_head^T`` (language.py:213-214)."""
        return lm_head.logits(hidden, self.weights.lm_head)

    def greedy(self, hidden: torch.Tensor, buffers: StepBuffers | None = None) -> torch.Tensor:
        """``logits(hidden).argmax(-1)`` without materialising the logits (decode_graph.py:167)."""
        if buffers is None:
            return lm_head.lm_head_argmax(hidden, self.weights.lm_head)[0]
        t = hidden.shape[0]
        return lm_head.lm_head_argmax(hidden, self.weights.lm_head, predicted=buffers.predicted[:t],
                                      workspace=buffers.head_workspace)[0]
