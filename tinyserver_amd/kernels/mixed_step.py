"""A continuous-batching step's two attention calls in one launch.

The reference's scheduler never puts prefill and decode sequences in one
batch (server/executor/scheduler.py:128-227); it runs a prefill batch's
forward (server/model/patches/qwen3.py:291-327) and then a decode batch's
(:328-416). An engine that runs both in one step calls ``mixed_step`` after
the prefill batch's ``qk_norm_rope_store``: it computes the prefill batch's
causal varlen attention and the decode batch's fused step (norm/RoPE + store
of each new token, then paged attention) in one kernel launch, plus the
decode merge. The outputs are bit-identical to ``flash_attn_varlen_func``
followed by ``paged_decode_step`` on one stream.
"""

from __future__ import annotations

import math

import torch

from .. import _lib
from .paged_attention import _workspace


def mixed_step(
    prefill_q: torch.Tensor,
    prefill_k: torch.Tensor,
    prefill_v: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_seqlen: int,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps: float,
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
    k, v, cu_seqlens_q = cu_seqlens_k and max_seqlen_q = max_seqlen_k, causal
    (the rotated q/k of the prefill tokens). q ... seq_lens: as
    ``paged_decode_step``'s arguments for the decode batch. The two batches
    must hold disjoint pages. One kernel runs both halves when the prefill is
    bf16/f16 with head_dim 128 and 4 q-heads per kv head, in the decode's
    dtype (each CU then runs one decode and one prefill workgroup); other
    shapes take the two launches, with the same results.
    """
    dev = _lib.require_device(prefill_q, prefill_k, prefill_v, cu_seqlens, q, k, v, q_weight, k_weight, cos, sin,
                              k_cache, v_cache, block_tables, seq_lens)
    if prefill_q.dim() != 3 or prefill_k.dim() != 3 or prefill_v.dim() != 3:
        raise ValueError("q, k, v must be 3D tensors")
    if prefill_q.shape[1] % prefill_k.shape[1] != 0:
        raise ValueError("num_heads_q must be divisible by num_heads_k for GQA")
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
        out = torch.empty_like(q)
    num_seqs, num_heads, head_dim = q.shape
    lib = _lib.load()
    stream = _lib.stream_of(dev)
    nbytes = int(lib.tsa_paged_decode_workspace_bytes(num_seqs, num_heads, k_cache.shape[1], head_dim,
                                                      block_tables.shape[1], k_cache.shape[2], num_workgroups))
    ws = _workspace(dev, stream, nbytes)
    vp = [_lib.view(t) for t in (prefill_out, prefill_q, prefill_k, prefill_v, cu_seqlens)]
    vd = [_lib.view(t) for t in (out, q, k, v, q_weight, k_weight, cos, sin)]
    vc = [_lib.view(t) for t in (k_cache, v_cache, block_tables, seq_lens)]
    rc = lib.tsa_mixed_step(
        *map(_lib.ref, vp),
        int(max_seqlen),
        float(prefill_scale),
        *map(_lib.ref, vd),
        float(eps),
        *map(_lib.ref, vc),
        1.0 / math.sqrt(head_dim),
        ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0,
        int(num_workgroups),
        int(prefill_workgroups),
        stream,
    )
    _lib.check(rc, "mixed_step")
    return prefill_out, out
