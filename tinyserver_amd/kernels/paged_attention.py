"""Paged decode attention -- drop-in for server/model/kernels/paged_attention.py.

``paged_attention_forward`` keeps the reference signature and its "3D"
ValueError (paged_attention.py:124-192). The output is allocated with
``torch.empty_like(query)`` as the reference does. The split-K partial-result
workspace is cached per (device, stream) and grown on demand.
"""

from __future__ import annotations

import math

import torch

from .. import _lib

_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def _key(device: torch.device, stream: int) -> tuple[int, int]:
    return (device.index if device.index is not None else torch.cuda.current_device(), stream)


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    ws = _workspaces.get(_key(device, stream))
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[_key(device, stream)] = ws
    return ws


def decode_workspace_bytes(num_seqs, num_heads, num_kv_heads, head_dim, max_blocks, block_size, num_workgroups=0):
    lib = _lib.load()
    return int(lib.tsa_paged_decode_workspace_bytes(num_seqs, num_heads, num_kv_heads, head_dim, max_blocks,
                                                    block_size, num_workgroups))


_WS_BYTES: dict[tuple, int] = {}


def _ws_bytes(device: torch.device, *shape) -> int:
    """tsa_paged_decode_workspace_bytes for a call shape, cached per device
    (the default grid depends on the device's CU count)."""
    key = (device.index, *shape)
    n = _WS_BYTES.get(key)
    if n is None:
        n = _WS_BYTES[key] = int(_lib.load().tsa_paged_decode_workspace_bytes(*shape))
    return n


def paged_attention_forward(
    query: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    block_size: int,
    seq_lens: torch.Tensor,
    *,
    num_workgroups: int = 0,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Decode-phase paged attention, one new token per sequence.

    ``out[s, h] = softmax(query[s, h] . K_s^T / sqrt(D)) V_s`` over the first
    ``seq_lens[s]`` tokens gathered through ``block_tables[s]``; q-head h reads
    kv head ``h // (Hq / Hkv)``. query: (B, Hq, D); caches (NB, Hkv, BS, D);
    block_tables (B, max_blocks) int32; seq_lens (B,) int32.
    ``num_workgroups`` (workgroups sharing the tile list; 0 = the library's
    choice, which for at most 64 (sequence, kv head) units with tables of at
    most 512 tokens is one workgroup per unit and no merge launch) and ``out``
    are extensions; the defaults reproduce the reference call.
    """
    if query.dim() != 3:
        raise ValueError(f"query must be a 3D tensor, but got shape {query.shape}")
    if k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError("k_cache and v_cache must be 4D tensors (num_blocks, num_kv_heads, block_size, head_dim)")
    if block_tables.dim() != 2:
        raise ValueError(f"block_tables must be a 2D tensor, but got shape {block_tables.shape}")
    if int(block_size) != k_cache.shape[2]:
        raise ValueError(f"block_size {block_size} does not match the cache's {k_cache.shape[2]}")
    dev = _lib.require_device(query, k_cache, v_cache, block_tables, seq_lens)
    if block_tables.dtype != torch.int32:
        block_tables = block_tables.to(torch.int32)
    if seq_lens.dtype != torch.int32:
        seq_lens = seq_lens.to(torch.int32)
    num_seqs, num_heads, head_dim = query.shape
    num_kv_heads = k_cache.shape[1]
    if out is None:
        out = torch.empty_like(query)
    softmax_scale = 1.0 / math.sqrt(head_dim)
    lib = _lib.load()
    stream = _lib.stream_of(dev)
    nbytes = _ws_bytes(dev, num_seqs, num_heads, num_kv_heads, head_dim, block_tables.shape[1], k_cache.shape[2],
                       int(num_workgroups))
    ws = _workspace(dev, stream, nbytes)
    views = [_lib.view(t) for t in (out, query, k_cache, v_cache, block_tables, seq_lens)]
    rc = lib.tsa_paged_decode(
        *map(_lib.ref, views),
        softmax_scale,
        ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0,
        int(num_workgroups),
        stream,
    )
    _lib.check(rc, "paged_attention_forward")
    return out


def paged_decode_step(
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
    num_workgroups: int = 0,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One decode step of the Qwen3 attention layer: QK RMSNorm + RoPE of the
    new token, its paged K/V store, and paged attention, in two launches.

    q (B, Hq, D), k and v (B, Hkv, D) are the raw projections of each
    sequence's new token, at position ``seq_lens[s] - 1``; cos/sin (B, D) are
    for those positions. Same results as ``qk_norm_rope_store`` followed by
    ``paged_attention_forward``. Raises NotImplementedError for shapes the
    fused kernel does not cover (head_dim != 128, fp32, pages not a multiple
    of 16 tokens, strided cache rows, more than 8 q-heads per kv head).
    """
    dev = _lib.require_device(q, k, v, q_weight, k_weight, cos, sin, k_cache, v_cache, block_tables, seq_lens)
    if block_tables.dtype != torch.int32:
        block_tables = block_tables.to(torch.int32)
    if seq_lens.dtype != torch.int32:
        seq_lens = seq_lens.to(torch.int32)
    num_seqs, num_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[1]
    if out is None:
        out = torch.empty_like(q)
    lib = _lib.load()
    stream = _lib.stream_of(dev)
    nbytes = _ws_bytes(dev, num_seqs, num_heads, num_kv_heads, head_dim, block_tables.shape[1], k_cache.shape[2],
                       int(num_workgroups))
    ws = _workspace(dev, stream, nbytes)
    v8 = [_lib.view(t) for t in (out, q, k, v, q_weight, k_weight, cos, sin)]
    v4 = [_lib.view(t) for t in (k_cache, v_cache, block_tables, seq_lens)]
    rc = lib.tsa_paged_decode_step(
        *map(_lib.ref, v8),
        float(eps),
        *map(_lib.ref, v4),
        1.0 / math.sqrt(head_dim),
        ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0,
        int(num_workgroups),
        stream,
    )
    _lib.check(rc, "paged_decode_step")
    return out
