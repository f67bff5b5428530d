"""Varlen causal prefill -- drop-in for server/model/kernels/varlen_attention.py.

``flash_attn_varlen_func`` keeps the reference signature, its ValueErrors and
its default scale (varlen_attention.py:145-218). q/k/v may be the strided
(T, H, D) views the call site builds (server/model/patches/qwen3.py:199-201);
only the innermost dimension must be unit-stride for the MFMA kernel (other
layouts take the generic kernel).
"""

from __future__ import annotations

import torch

from .. import _lib


def flash_attn_varlen_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    causal: bool,
    softmax_scale: float | None = None,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Per sequence b and q-head h: softmax(q k^T * scale) v over keys
    cu_seqlens_k[b]..cu_seqlens_k[b+1]; causal masks key j > query i within
    the sequence (top-left aligned, as the reference kernel does)."""
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k, v must be 3D tensors")
    _, num_heads_q, head_dim = q.shape
    num_heads_k = k.shape[1]
    if num_heads_q % num_heads_k != 0:
        raise ValueError("num_heads_q must be divisible by num_heads_k for GQA")
    if softmax_scale is None:
        softmax_scale = 1.0 / (head_dim**0.5)
    dev = _lib.require_device(q, k, v, cu_seqlens_q, cu_seqlens_k)
    if cu_seqlens_q.dtype != torch.int32:
        cu_seqlens_q = cu_seqlens_q.to(torch.int32)
    if cu_seqlens_k.dtype != torch.int32:
        cu_seqlens_k = cu_seqlens_k.to(torch.int32)
    if out is None:
        out = torch.empty_like(q)
    lib = _lib.load()
    views = [_lib.view(t) for t in (out, q, k, v, cu_seqlens_q, cu_seqlens_k)]
    rc = lib.tsa_varlen_prefill(
        *map(_lib.ref, views),
        int(max_seqlen_q),
        int(max_seqlen_k),
        1 if causal else 0,
        float(softmax_scale),
        _lib.stream_of(dev),
    )
    _lib.check(rc, "flash_attn_varlen_func")
    return out
