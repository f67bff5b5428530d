"""A continuous-batching step's two attention calls in one launch.

The reference's scheduler never puts prefill and decode sequences in one
batch (server/executor/scheduler.py:128-227); it runs a prefill batch's
forward, whose attention is ``flash_attn_varlen_func``
(server/model/patches/qwen3.py:173-214), and then a decode batch's, whose
attention is ``paged_attention_forward`` (:387-409). An engine that runs
both batches in one step stores every new token's K/V first (one
``qk_norm_rope_store`` over the tokens of both) and then calls
``mixed_attention``: both attentions in one kernel launch, plus the decode
merge. The outputs are bit-identical to the two calls on one stream.
"""

from __future__ import annotations

import math

import torch

from .. import _lib
from .paged_attention import _workspace, _ws_bytes


def mixed_attention(
    prefill_q: torch.Tensor,
    prefill_k: torch.Tensor,
    prefill_v: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_seqlen: int,
    query: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    prefill_scale: float | None = None,
    num_workgroups: int = 0,
    prefill_workgroups: int = 0,
    prefill_out: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (prefill attention (T, Hq, D), decode attention (B, Hq, D)).

    prefill_q/k/v, cu_seqlens, max_seqlen: as ``flash_attn_varlen_func``'s q,
    k, v, cu_seqlens_q = cu_seqlens_k and max_seqlen_q = max_seqlen_k, causal.
    query ... seq_lens: as ``paged_attention_forward``'s arguments (the
    decode tokens' K/V already in the cache), scale head_dim^-1/2. One kernel
    can run both halves when the decode has head_dim 128, pages a multiple
    of 16 tokens and contiguous cache rows, and the prefill is bf16/f16 with
    head_dim 128 and 4 q-heads per kv head, in the decode's dtype (each CU
    then runs one decode and one prefill workgroup). ``prefill_workgroups``
    > 0 asks for it with that many prefill workgroups; 0 takes it when the
    prefill batch has at most 512 tokens and the decode's block tables span
    at most 131072 tokens (batch x table width x page size): both halves
    small, where it is faster. Otherwise the two launches. Same results
    either way.
    """
    if prefill_q.dim() != 3 or prefill_k.dim() != 3 or prefill_v.dim() != 3:
        raise ValueError("q, k, v must be 3D tensors")
    if prefill_q.shape[1] % prefill_k.shape[1] != 0:
        raise ValueError("num_heads_q must be divisible by num_heads_k for GQA")
    if query.dim() != 3:
        raise ValueError("query must be 3D tensor (num_seqs, num_heads, head_dim)")
    if k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError("k_cache and v_cache must be 4D tensors (num_blocks, num_kv_heads, block_size, head_dim)")
    if block_tables.dim() != 2:
        raise ValueError(f"block_tables must be a 2D tensor, but got shape {block_tables.shape}")
    if cu_seqlens.dim() != 1:
        raise ValueError("cu_seqlens must be a 1D tensor")
    dev = _lib.require_device(prefill_q, prefill_k, prefill_v, cu_seqlens, query, k_cache, v_cache, block_tables,
                              seq_lens)
    if prefill_scale is None:
        prefill_scale = 1.0 / (prefill_q.shape[2] ** 0.5)
    if cu_seqlens.dtype != torch.int32:
        cu_seqlens = cu_seqlens.to(torch.int32)
    if block_tables.dtype != torch.int32:
        block_tables = block_tables.to(torch.int32)
    if seq_lens.dtype != torch.int32:
        seq_lens = seq_lens.to(torch.int32)
    if prefill_out is None:
        prefill_out = torch.empty_like(prefill_q)
    if out is None:
        out = torch.empty_like(query)
    num_seqs, num_heads, head_dim = query.shape
    lib = _lib.load()
    stream = _lib.stream_of(dev)
    nbytes = _ws_bytes(dev, num_seqs, num_heads, k_cache.shape[1], head_dim, block_tables.shape[1], k_cache.shape[2],
                       int(num_workgroups))
    ws = _workspace(dev, stream, nbytes)
    vp = [_lib.view(t) for t in (prefill_out, prefill_q, prefill_k, prefill_v, cu_seqlens)]
    vd = [_lib.view(t) for t in (out, query, k_cache, v_cache, block_tables, seq_lens)]
    rc = lib.tsa_mixed_attention(
        *map(_lib.ref, vp),
        int(max_seqlen),
        float(prefill_scale),
        *map(_lib.ref, vd),
        1.0 / math.sqrt(head_dim),
        ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0,
        int(num_workgroups),
        int(prefill_workgroups),
        stream,
    )
    _lib.check(rc, "mixed_attention")
    return prefill_out, out
