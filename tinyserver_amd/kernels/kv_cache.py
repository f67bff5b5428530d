"""Paged K/V store -- drop-in for server/model/kernels/kv_cache.py.

``store_kv_cache`` and ``store_kv_cache_batched`` keep the reference's
signatures and ValueError guards (kv_cache.py:73-119, 194-251);
``store_kv_cache_paged`` computes each token's (block, slot) on the device
from the per-sequence block tables, replacing the per-token Python mapping
loop and per-sequence launch loop at server/model/patches/qwen3.py:296-318
and :335-357.
"""

from __future__ import annotations

import torch

from .. import _lib


def _src_like_cache(src: torch.Tensor, cache: torch.Tensor) -> torch.Tensor:
    # The reference's Triton store converts to the cache dtype on store.
    return src if src.dtype == cache.dtype else src.to(cache.dtype)


def store_kv_cache(
    start_position: int,
    block_table: torch.Tensor,
    k_src: torch.Tensor,
    v_src: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
) -> None:
    """Scatter one sequence's new K/V (Hkv, n, D) into the paged cache.

    Token i lands at absolute position start_position + i:
    ``cache[block_table[p // BS], h, p % BS, :]`` (kv_cache.py:73-119).
    """
    if k_src.dim() != 3 or v_src.dim() != 3:
        raise ValueError(f"k_src and v_src must be 3D tensors, but got shapes {k_src.shape} and {v_src.shape}")
    dev = _lib.require_device(k_src, v_src, k_cache, v_cache, block_table)
    if block_table.dtype != torch.int32:
        block_table = block_table.to(torch.int32)
    lib = _lib.load()
    k_src, v_src = _src_like_cache(k_src, k_cache), _src_like_cache(v_src, v_cache)
    views = [_lib.view(t) for t in (k_src, v_src, k_cache, v_cache, block_table)]
    rc = lib.tsa_store_kv(*map(_lib.ref, views), int(start_position), _lib.stream_of(dev))
    _lib.check(rc, "store_kv_cache")


def store_kv_cache_batched(
    k_src: torch.Tensor,
    v_src: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_mapping: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """``cache[block_mapping[t], h, slot_mapping[t], :] = src[h, t, :]`` (kv_cache.py:194-251)."""
    if k_src.dim() != 3 or v_src.dim() != 3:
        raise ValueError(f"k_src and v_src must be 3D tensors, but got shapes {k_src.shape} and {v_src.shape}")
    if k_src.shape != v_src.shape:
        raise ValueError(f"k_src and v_src must have the same shape, but got {k_src.shape} and {v_src.shape}")
    num_tokens = k_src.shape[1]
    if block_mapping.shape[0] != num_tokens or slot_mapping.shape[0] != num_tokens:
        raise ValueError(
            f"block_mapping and slot_mapping must have length num_tokens ({num_tokens}), "
            f"but got {block_mapping.shape[0]} and {slot_mapping.shape[0]}"
        )
    dev = _lib.require_device(k_src, v_src, k_cache, v_cache, block_mapping, slot_mapping)
    lib = _lib.load()
    k_src, v_src = _src_like_cache(k_src, k_cache), _src_like_cache(v_src, v_cache)
    views = [_lib.view(t) for t in (k_src, v_src, k_cache, v_cache, block_mapping, slot_mapping)]
    rc = lib.tsa_store_kv_mapped(*map(_lib.ref, views), _lib.stream_of(dev))
    _lib.check(rc, "store_kv_cache_batched")


def store_kv_cache_paged(
    k_src: torch.Tensor,
    v_src: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    cu_seqlens: torch.Tensor,
    positions: torch.Tensor | None = None,
) -> None:
    """Store a packed batch with device-side addressing.

    k_src, v_src: (Hkv, T, D) -- any strides, so the (T, Hkv, D) projection
    output is passed as ``k.transpose(0, 1)`` without a copy. Tokens of
    sequence s are ``cu_seqlens[s]:cu_seqlens[s+1]``; token t sits at
    ``positions[t]`` (decode) or at ``t - cu_seqlens[s]`` (prefill, positions
    None) and goes to ``cache[block_tables[s, p // BS], h, p % BS, :]``.
    """
    if k_src.dim() != 3 or v_src.dim() != 3:
        raise ValueError(f"k_src and v_src must be 3D tensors, but got shapes {k_src.shape} and {v_src.shape}")
    if k_src.shape != v_src.shape:
        raise ValueError(f"k_src and v_src must have the same shape, but got {k_src.shape} and {v_src.shape}")
    if block_tables.dim() != 2 or cu_seqlens.dim() != 1 or cu_seqlens.shape[0] != block_tables.shape[0] + 1:
        raise ValueError("block_tables must be (num_seqs, max_blocks) and cu_seqlens (num_seqs + 1,)")
    if positions is not None and positions.shape[0] != k_src.shape[1]:
        raise ValueError(f"positions must have num_tokens ({k_src.shape[1]}) entries, got {positions.shape[0]}")
    dev = _lib.require_device(k_src, v_src, k_cache, v_cache, block_tables, cu_seqlens, positions)
    lib = _lib.load()
    k_src, v_src = _src_like_cache(k_src, k_cache), _src_like_cache(v_src, v_cache)
    views = [_lib.view(t) for t in (k_src, v_src, k_cache, v_cache, block_tables, cu_seqlens, positions)]
    rc = lib.tsa_store_kv_paged(*map(_lib.ref, views), _lib.stream_of(dev))
    _lib.check(rc, "store_kv_cache_paged")
