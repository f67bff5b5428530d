"""Paged K/V store and gather, restated on the CPU (test infrastructure).

The reference writes new K/V rows into a paged pool laid out
``(num_blocks, num_kv_heads, block_size, head_dim)`` per layer
(server/model/patches/qwen3.py:49-62). A token at absolute position ``p`` of a
sequence with block table ``bt`` lands at ``cache[bt[p // BS], h, p % BS, :]``.
The restatement is plain index assignment -- the reference's Triton store
kernels are exact copies, so the oracle is bit-exact by construction.
"""

from __future__ import annotations

import torch


def store_kv_cache(start_position, block_table, k_src, v_src, k_cache, v_cache) -> None:
    """store_kv_cache / _store_kv_kernel (server/model/kernels/kv_cache.py:6-70, 73-119).

    k_src, v_src: (Hkv, n, D). Token i goes to absolute position
    start_position + i (kv_cache.py:41-53).
    """
    if k_src.dim() != 3 or v_src.dim() != 3:
        raise ValueError(f"k_src and v_src must be 3D tensors, but got shapes {k_src.shape} and {v_src.shape}")
    bt = [int(b) for b in block_table.tolist()]
    block_size = k_cache.shape[2]
    for t in range(k_src.shape[1]):
        pos = int(start_position) + t
        blk = bt[pos // block_size]  # kv_cache.py:47-50
        slot = pos % block_size  # kv_cache.py:53
        k_cache[blk, :, slot, :] = k_src[:, t, :]  # kv_cache.py:55-62
        v_cache[blk, :, slot, :] = v_src[:, t, :]


def store_kv_cache_batched(k_src, v_src, k_cache, v_cache, block_mapping, slot_mapping) -> None:
    """store_kv_cache_batched (server/model/kernels/kv_cache.py:122-191, 194-251).

    ``cache[block_mapping[t], h, slot_mapping[t], :] = src[h, t, :]`` for every
    token t, with the reference's argument guards (kv_cache.py:210-234).
    """
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
    blk = block_mapping.to(torch.int64)
    slot = slot_mapping.to(torch.int64)
    # Advanced indexing (blk[t], :, slot[t], :) -> (T, Hkv, D); src is (Hkv, T, D).
    k_cache[blk, :, slot, :] = k_src.transpose(0, 1).to(k_cache.dtype)
    v_cache[blk, :, slot, :] = v_src.transpose(0, 1).to(v_cache.dtype)


def build_block_slot_mappings(sequences, block_size: int, start_positions=None):
    """The prefill mapping loop (server/model/patches/qwen3.py:296-303).

    ``sequences`` is the InferenceContext list of ``{"num_tokens", "block_table"}``.
    Prefill always starts at position 0 at the call site; ``start_positions``
    generalises to the reference test helper's rule
    (tests/model/test_kv_cache_kernels.py:16-37). Returns int64 tensors.
    """
    block_mapping, slot_mapping = [], []
    for i, seq in enumerate(sequences):
        bt = seq["block_table"]
        p0 = 0 if start_positions is None else int(start_positions[i])
        for j in range(int(seq["num_tokens"])):
            p = p0 + j
            block_mapping.append(int(bt[p // block_size]))
            slot_mapping.append(p % block_size)
    return (torch.tensor(block_mapping, dtype=torch.int64), torch.tensor(slot_mapping, dtype=torch.int64))


def gather_kv_cache(next_position: int, block_table, k_cache, v_cache):
    """gather_kv_cache (server/model/patches/qwen3.py:423-466): the inverse of the store.

    Returns (Hkv, next_position + 1, D) K and V for one sequence.
    """
    block_size = k_cache.shape[2]
    seq_len = int(next_position) + 1
    bt = [int(b) for b in block_table]
    idx = torch.arange(seq_len)
    blocks = torch.tensor([bt[i // block_size] for i in range(seq_len)], dtype=torch.int64)
    slots = idx % block_size
    k_full = k_cache[blocks, :, slots, :].transpose(0, 1).contiguous()
    v_full = v_cache[blocks, :, slots, :].transpose(0, 1).contiguous()
    return k_full, v_full


def gather_kv_cache_loop(next_position: int, block_table, k_cache, v_cache):
    """gather_kv_cache as the reference writes it: one Python step per token
    (server/model/patches/qwen3.py:444-466). Used as the literal CPU baseline."""
    block_size = k_cache.shape[2]
    seq_len = next_position + 1
    k_full = torch.empty((k_cache.shape[1], seq_len, k_cache.shape[3]), dtype=k_cache.dtype)
    v_full = torch.empty((v_cache.shape[1], seq_len, v_cache.shape[3]), dtype=v_cache.dtype)
    for i in range(seq_len):
        block_idx = block_table[i // block_size]
        pos_in_block = i % block_size
        k_full[:, i, :] = k_cache[block_idx, :, pos_in_block, :]
        v_full[:, i, :] = v_cache[block_idx, :, pos_in_block, :]
    return k_full, v_full
