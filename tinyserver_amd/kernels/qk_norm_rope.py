"""Fused Qwen3 QK RMSNorm + rotate-half RoPE (+ optional paged K/V store).

Replaces the eager calls at server/model/patches/qwen3.py:268-287 --
``q_norm``/``k_norm`` (transformers modeling_qwen3.py:59-64) and
``apply_rotary_pos_emb`` (:148-170) -- with one kernel that keeps HF's rounding
points in the model dtype. Inputs are the head-split projection outputs,
token-major: q (T, Hq, D), k (T, Hkv, D) (a leading batch dim of 1 is
accepted); cos/sin are HF's position embeddings, (T, D) or (1, T, D).
Outputs are token-major (T, H, D) -- the layout paged decode and varlen
prefill consume directly.
"""

from __future__ import annotations

import torch

from .. import _lib


def _tokens_major(x: torch.Tensor, name: str) -> torch.Tensor:
    if x.dim() == 4 and x.shape[0] == 1:
        x = x[0]
    if x.dim() != 3:
        raise ValueError(f"{name} must be (T, H, D) or (1, T, H, D), got shape {tuple(x.shape)}")
    return x


def _table(x: torch.Tensor, name: str) -> torch.Tensor:
    if x.dim() == 3 and x.shape[0] == 1:
        x = x[0]
    if x.dim() != 2:
        raise ValueError(f"{name} must be (T, D) or (1, T, D), got shape {tuple(x.shape)}")
    return x


def qk_norm_rope(q, k, q_weight, k_weight, cos, sin, eps, *, q_out=None, k_out=None):
    """Return (q_rot (T, Hq, D), k_rot (T, Hkv, D))."""
    q, k = _tokens_major(q, "q"), _tokens_major(k, "k")
    cos, sin = _table(cos, "cos"), _table(sin, "sin")
    dev = _lib.require_device(q, k, q_weight, k_weight, cos, sin)
    q_out = torch.empty(q.shape, dtype=q.dtype, device=dev) if q_out is None else q_out
    k_out = torch.empty(k.shape, dtype=k.dtype, device=dev) if k_out is None else k_out
    lib = _lib.load()
    views = [_lib.view(t) for t in (q, k, q_out, k_out, q_weight, k_weight, cos, sin)]
    rc = lib.tsa_qk_norm_rope(*map(_lib.ref, views), float(eps), _lib.stream_of(dev))
    _lib.check(rc, "qk_norm_rope")
    return q_out, k_out


def qk_norm_rope_store(
    q, k, v, q_weight, k_weight, cos, sin, eps, k_cache, v_cache, block_tables, cu_seqlens, positions=None,
    *, q_out=None, k_out=None, return_k=True,
):
    """Norm + RoPE q and k, and store the rotated K and raw V into the paged
    cache with device-side addressing (tokens of sequence s are
    cu_seqlens[s]:cu_seqlens[s+1], at positions[t] or t - cu_seqlens[s]).
    Returns (q_rot, k_rot or None)."""
    q, k, v = _tokens_major(q, "q"), _tokens_major(k, "k"), _tokens_major(v, "v")
    cos, sin = _table(cos, "cos"), _table(sin, "sin")
    dev = _lib.require_device(q, k, v, q_weight, k_weight, cos, sin, k_cache, v_cache, block_tables, cu_seqlens,
                              positions)
    q_out = torch.empty(q.shape, dtype=q.dtype, device=dev) if q_out is None else q_out
    if return_k and k_out is None:
        k_out = torch.empty(k.shape, dtype=k.dtype, device=dev)
    lib = _lib.load()
    views = [_lib.view(t) for t in (q, k, v, q_out, k_out, q_weight, k_weight, cos, sin)]
    store = [_lib.view(t) for t in (k_cache, v_cache, block_tables, cu_seqlens, positions)]
    rc = lib.tsa_qk_norm_rope_store(*map(_lib.ref, views), float(eps), *map(_lib.ref, store), _lib.stream_of(dev))
    _lib.check(rc, "qk_norm_rope_store")
    return q_out, k_out
