"""Attention on gfx950: the drop-ins for attention.paged_extend (oxr_runtime/attention.py:96-109),
attention.paged_decode (attention.py:76-93) and attention.varlen (attention.py:47-59).

The paged entry points run csrc/paged_attention.hip (MFMA QK^T and PV tiles, context split across
8-wave workgroups merged on chip, then a small log-sum-exp merge of the splits); ``varlen`` runs
csrc/varlen_attention.hip (key tiles staged in LDS and shared by 128 query rows).  The vision
entry points (``varlen_bidirectional`` with head dim 72, ``rotary``) are outside this build.
"""

from __future__ import annotations

import torch

from . import _lib
from .gemm import PackedMatrix


def workspace_bytes(batch: int, num_kv_heads: int, max_seq_len: int) -> int:
    return int(_lib.lib().oxr_paged_extend_workspace_bytes(batch, num_kv_heads, max_seq_len))


def plan_ints(batch: int, tokens_per_seq: int, num_heads: int, num_kv_heads: int, max_seq_len: int) -> int:
    """int32 entries of a context-piece plan (:func:`build_plan`) for these launch parameters; 0 when
    the launch keeps every context in one piece."""
    return int(_lib.lib().oxr_paged_extend_plan_ints(batch, tokens_per_seq, num_heads, num_kv_heads, max_seq_len))


def build_plan(seq_lens: torch.Tensor, tokens_per_seq: int, num_heads: int, num_kv_heads: int, max_seq_len: int,
               *, out: torch.Tensor | None = None) -> torch.Tensor | None:
    """Balanced context pieces for a :func:`paged_extend` / :func:`qk_norm_rope_paged_extend` launch over
    ``seq_lens`` (device int32 [B]), written on the device (so under graph capture it follows the
    lengths of each replay).  Without a plan every context is cut into the same number of pieces and
    the longest context bounds the launch; with one, pieces are about the batch's mean share and long
    contexts take the workgroups short ones leave.  Pass the result as ``plan=`` to a launch with the
    same lengths, batch, tokens_per_seq, heads and max_seq_len.  None when no plan is needed."""
    device = _lib.require_gpu(seq_lens, name="build_plan")
    _lib.require(seq_lens.dtype == torch.int32 and seq_lens.dim() == 1 and seq_lens.is_contiguous(),
                 "seq_lens must be contiguous int32 [B]")
    b = seq_lens.shape[0]
    n = plan_ints(b, tokens_per_seq, num_heads, num_kv_heads, max_seq_len)
    if n == 0:
        return None
    if out is None:
        out = torch.empty(n, dtype=torch.int32, device=device)
    _lib.require(out.dtype == torch.int32 and out.is_contiguous() and out.numel() >= n, "build_plan: out too small")
    _lib.call("oxr_paged_extend_plan", seq_lens.data_ptr(), b, tokens_per_seq, num_heads, num_kv_heads, max_seq_len,
              out.data_ptr(), out.numel(), _lib.stream(device))
    return out


def paged_extend(
    q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, seq_lens: torch.Tensor,
    block_table: torch.Tensor, *, scale: float | None = None, max_seq_len: int | None = None,
    out: torch.Tensor | None = None, workspace: torch.Tensor | None = None, plan: torch.Tensor | None = None,
) -> torch.Tensor:
    """Each sequence brings S new tokens (``q`` is ``[B, S, heads, dim]``; their K/V are already in the
    paged cache); token j sees itself and everything before it (``seq_lens`` includes the S tokens).
    Returns ``[B, S, heads, dim]``.

    ``max_seq_len`` bounds every ``seq_lens[b]`` (default: the block table's span) and sizes the
    context split; ``out`` and ``workspace`` (bytes from :func:`workspace_bytes`) may be passed in to
    avoid allocations; ``plan`` (from :func:`build_plan`) balances contexts of different lengths."""
    device = _lib.require_gpu(q, k_cache, v_cache, seq_lens, block_table, name="paged_extend")
    _lib.require(q.dim() == 4 and q.dtype == torch.bfloat16 and q.is_contiguous(), "q must be contiguous bf16 [B, S, H, D]")
    b, s, h, d = q.shape
    _lib.require(k_cache.dim() == 4 and k_cache.shape == v_cache.shape, "caches must be [blocks, block_size, KV, D]")
    _lib.require(k_cache.dtype == torch.bfloat16 and v_cache.dtype == torch.bfloat16, "caches must be bf16")
    _lib.require(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    num_blocks, block_size, kv, dk = k_cache.shape
    _lib.require(dk == d, "head_dim of q and caches differ")
    _lib.require(seq_lens.dtype == torch.int32 and seq_lens.shape == (b,), "seq_lens must be int32 [B]")
    _lib.require(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] >= b,
                 "block_table must be int32 [>=B, W]")
    _lib.require(block_table.stride(1) == 1, "block_table rows must be contiguous")
    if max_seq_len is None:
        max_seq_len = block_table.shape[1] * block_size
    if scale is None:
        scale = d ** -0.5
    if out is None:
        out = torch.empty_like(q)
    need = workspace_bytes(b, kv, max_seq_len)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
    _lib.require(workspace.numel() * workspace.element_size() >= need, "paged_extend: workspace too small")
    args = (q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), seq_lens.data_ptr(), block_table.data_ptr(),
            block_table.stride(0), b, s, h, kv, d, block_size, num_blocks, max_seq_len, float(scale), out.data_ptr(),
            workspace.data_ptr(), workspace.numel() * workspace.element_size())
    if plan is None:
        _lib.call("oxr_paged_extend", *args, _lib.stream(device))
    else:
        _check_plan(plan, b, s, h, kv, max_seq_len, device)
        _lib.call("oxr_paged_extend_planned", *args, plan.data_ptr(), plan.numel(), _lib.stream(device))
    return out


def _check_plan(plan: torch.Tensor, b: int, s: int, h: int, kv: int, max_seq_len: int, device) -> None:
    _lib.require(plan.device == device and plan.dtype == torch.int32 and plan.is_contiguous()
                 and plan.numel() >= plan_ints(b, s, h, kv, max_seq_len), "plan: int32 from build_plan for this launch")


def varlen(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor, max_len: int, *, causal: bool,
    scale: float | None = None, out: torch.Tensor | None = None,
) -> torch.Tensor:
    """The drop-in for attention.varlen (oxr_runtime/attention.py:47-59): sequences concatenated along
    the token axis (``q`` ``[T, heads, 128]``, ``k``/``v`` ``[T, kv_heads, 128]``, ``cu_seqlens`` int32
    ``[n + 1]``), attention within each sequence, causal or not.  Returns ``[T, heads, 128]``."""
    device = _lib.require_gpu(q, k, v, cu_seqlens, name="varlen")
    _lib.require(q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16,
                 "varlen: bf16 q, k, v required")
    _lib.require(q.dim() == 3 and k.dim() == 3 and k.shape == v.shape and q.shape[0] == k.shape[0]
                 and q.shape[2] == k.shape[2], "varlen: q [T, H, D], k and v [T, KV, D]")
    _lib.require(q.is_contiguous() and k.is_contiguous() and v.is_contiguous(), "varlen: contiguous q, k, v")
    _lib.require(cu_seqlens.dtype == torch.int32 and cu_seqlens.dim() == 1 and cu_seqlens.is_contiguous(),
                 "varlen: cu_seqlens must be contiguous int32 [n + 1]")
    t, h, d = q.shape
    if scale is None:
        scale = d ** -0.5
    if out is None:
        out = torch.empty_like(q)
    _lib.require(out.shape == q.shape and out.dtype == torch.bfloat16 and out.is_contiguous(), "varlen: out like q")
    _lib.call("oxr_varlen_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), cu_seqlens.data_ptr(),
              cu_seqlens.shape[0] - 1, int(max_len), h, k.shape[1], d, 1 if causal else 0, float(scale),
              out.data_ptr(), _lib.stream(device))
    return out


def paged_decode(
    q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, seq_lens: torch.Tensor,
    block_table: torch.Tensor, *, scale: float | None = None, max_seq_len: int | None = None,
    out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """The drop-in for attention.paged_decode (oxr_runtime/attention.py:76-93): one new token per
    sequence (``q`` is ``[B, heads, dim]``, its K/V already in the paged cache; ``seq_lens`` includes
    it) attending to every key of its sequence.  Returns ``[B, heads, dim]``.  The same kernels as
    :func:`paged_extend` with one token per sequence."""
    _lib.require(q.dim() == 3, "q must be [B, H, D]")
    b, h, d = q.shape
    if out is not None:
        _lib.require(out.shape == q.shape and out.is_contiguous(), "out must be contiguous [B, H, D]")
        out = out.view(b, 1, h, d)
    res = paged_extend(q.view(b, 1, h, d), k_cache, v_cache, seq_lens, block_table, scale=scale,
                       max_seq_len=max_seq_len, out=out, workspace=workspace)
    return res.view(b, h, d)


def qk_norm_rope_paged_extend(
    qkv: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor, cos_table: torch.Tensor,
    sin_table: torch.Tensor, positions: torch.Tensor, eps: float, k_cache: torch.Tensor, v_cache: torch.Tensor,
    slots: torch.Tensor, seq_lens: torch.Tensor, block_table: torch.Tensor, num_heads: int, *,
    scale: float | None = None, max_seq_len: int | None = None, out: torch.Tensor | PackedMatrix | None = None,
    workspace: torch.Tensor | None = None, plan: torch.Tensor | None = None,
) -> torch.Tensor | PackedMatrix:
    """The decoder layer's attention block of the verify step (oxr_runtime/language.py:311-316) in one
    launch: ``kernels.qk_norm_rope_store`` (q/k RMSNorm + RoPE at ``positions``, K/V into the cache at
    ``slots``) followed by :func:`paged_extend`, with q kept on chip.  ``qkv`` is ``[B*S, (H+2KV)*D]``
    for the S new tokens of each of the B sequences; returns ``[B, S, H, D]`` (or fills ``out``
    given as a packed ``[B*S, H*D]`` :class:`~.gemm.PackedMatrix`, the o_proj GEMM's x) and leaves
    the cache rows exactly as the two separate calls would."""
    device = _lib.require_gpu(qkv, q_weight, k_weight, cos_table, sin_table, positions, k_cache, v_cache, slots,
                              seq_lens, block_table, name="qk_norm_rope_paged_extend")
    _lib.require(qkv.dtype == torch.bfloat16 and qkv.dim() == 2 and qkv.is_contiguous(), "qkv must be contiguous bf16")
    _lib.require(k_cache.dim() == 4 and k_cache.shape == v_cache.shape, "caches must be [blocks, block_size, KV, D]")
    _lib.require(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    num_blocks, block_size, kv, d = k_cache.shape
    b = seq_lens.shape[0]
    n = qkv.shape[0]
    _lib.require(b > 0 and n % b == 0 and qkv.shape[1] == (num_heads + 2 * kv) * d, "qkv shape mismatch")
    s = n // b
    _lib.require(positions.dtype == torch.int64 and positions.shape == (n,), "positions must be int64 [B*S]")
    _lib.require(slots.dtype == torch.int64 and slots.shape == (n,), "slots must be int64 [B*S]")
    _lib.require(seq_lens.dtype == torch.int32 and block_table.dtype == torch.int32 and block_table.stride(1) == 1,
                 "seq_lens / block_table must be int32, table rows contiguous")
    _lib.require(cos_table.dim() == 2 and cos_table.shape == sin_table.shape and cos_table.shape[1] == d // 2,
                 "cos/sin tables must be [rows, D/2]")
    if max_seq_len is None:
        max_seq_len = block_table.shape[1] * block_size
    if scale is None:
        scale = d ** -0.5
    if out is None:
        out = torch.empty(b, s, num_heads, d, dtype=torch.bfloat16, device=device)
    packed = isinstance(out, PackedMatrix)
    if packed:
        _lib.require(out.shape == (n, num_heads * d) and out.data.numel() >= -(-n // 16) * 16 * num_heads * d,
                     "qk_norm_rope_paged_extend: packed out must be [B*S, H*D]")
    else:
        _lib.require(out.shape == (b, s, num_heads, d) and out.is_contiguous(), "out must be contiguous [B, S, H, D]")
    out_t = out.data if packed else out
    need = workspace_bytes(b, kv, max_seq_len)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
    args = (qkv.data_ptr(), q_weight.data_ptr(), k_weight.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(),
            cos_table.shape[0], positions.data_ptr(), float(eps), k_cache.data_ptr(), v_cache.data_ptr(),
            slots.data_ptr(), num_blocks * block_size, seq_lens.data_ptr(), block_table.data_ptr(),
            block_table.stride(0), b, s, num_heads, kv, d, block_size, num_blocks, max_seq_len, float(scale),
            out_t.data_ptr(), 1 if packed else 0, workspace.data_ptr(), workspace.numel() * workspace.element_size())
    if plan is None:
        _lib.call("oxr_qk_norm_rope_paged_extend", *args, _lib.stream(device))
    else:
        _check_plan(plan, b, s, num_heads, kv, max_seq_len, device)
        _lib.call("oxr_qk_norm_rope_paged_extend_planned", *args, plan.data_ptr(), plan.numel(), _lib.stream(device))
    return out
