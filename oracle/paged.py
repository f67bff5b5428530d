"""Paged decode attention, restated on the CPU (test infrastructure).

Two restatements of the reference:

* ``paged_attention_forward`` -- the Triton kernel's algorithm
  (server/model/kernels/paged_attention.py:8-121): per (sequence, q-head), an
  fp32 online softmax walked one logical block at a time through the block
  table, GQA kv head = h // (Hq / Hkv), slots past ``seq_len`` scored -inf and
  loaded as 0, output = acc / l cast to the query dtype. Vectorised here over
  sequences and heads; sequences whose blocks have run out see only -inf
  scores, which leave (m, l, acc) unchanged.
* ``decode_cpu_path`` -- the reference's CPU decode branch
  (server/model/patches/qwen3.py:359-385): per sequence, gather K/V with the
  per-token loop of gather_kv_cache, repeat_interleave the kv heads and call
  SDPA. This is the literal CPU path timed as the CPU baseline.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .kv_store import gather_kv_cache, gather_kv_cache_loop


def paged_attention_forward(query, k_cache, v_cache, block_tables, block_size, seq_lens):
    """paged_attention_forward (paged_attention.py:124-192) + its kernel (:8-121)."""
    if query.dim() != 3:
        raise ValueError(f"query must be a 3D tensor, but got shape {query.shape}")
    num_seqs, num_heads, head_dim = query.shape
    num_kv_heads = k_cache.shape[1]
    group = num_heads // num_kv_heads  # paged_attention.py:54
    kv_head = torch.arange(num_heads) // group  # paged_attention.py:55
    scale = 1.0 / math.sqrt(head_dim)  # paged_attention.py:170

    q = query.to(torch.float32)  # :66
    seq_lens = seq_lens.to(torch.int64)
    n_blocks = (seq_lens + block_size - 1) // block_size  # :70
    m = torch.full((num_seqs, num_heads), float("-inf"))  # :73
    l = torch.zeros((num_seqs, num_heads))  # :74
    acc = torch.zeros((num_seqs, num_heads, head_dim))  # :75
    slots = torch.arange(block_size)
    max_blocks = int(n_blocks.max()) if num_seqs else 0
    for b in range(max_blocks):  # :77
        active = b < n_blocks  # (S,) sequences that still have a block b
        phys = block_tables[:, b].to(torch.int64).clone()  # :78-80
        phys[~active] = 0  # never dereference the padded tail for finished sequences
        tok = b * block_size + slots  # :102
        valid = (tok[None, :] < seq_lens[:, None]) & active[:, None]  # (S, BS), :88
        k = k_cache[phys].to(torch.float32)[:, kv_head]  # (S, Hq, BS, D), :82-92
        v = v_cache[phys].to(torch.float32)[:, kv_head]
        k = torch.where(valid[:, None, :, None], k, 0.0)  # masked load, other=0
        v = torch.where(valid[:, None, :, None], v, 0.0)
        qk = (q[:, :, None, :] * k).sum(-1) * scale  # :99-100
        qk = torch.where(valid[:, None, :], qk, float("-inf"))  # :103-105
        m_new = torch.maximum(m, qk.max(-1).values)  # :107
        p = torch.exp(qk - m_new[..., None])  # :108
        alpha = torch.exp(m - m_new)  # :109
        # A sequence with no block b has qk = -inf everywhere: p = 0, alpha = 1.
        alpha = torch.where(active[:, None], alpha, 1.0)
        p = torch.where(active[:, None, None], p, 0.0)
        acc = acc * alpha[..., None] + (p[..., None] * v).sum(-2)  # :110-111
        l = l * alpha + p.sum(-1)  # :112
        m = torch.where(active[:, None], m_new, m)  # :113
    return (acc / l[..., None]).to(query.dtype)  # :115-121


def decode_cpu_path(q, k_cache, v_cache, block_tables, positions, literal_gather: bool = True):
    """The reference's CPU decode branch (server/model/patches/qwen3.py:359-385).

    q: (1, Hq, B, D) rotated queries; block_tables: list of per-sequence lists;
    positions: (B,) absolute position of each sequence's new token (already
    stored). Returns (B, Hq, D). ``literal_gather`` selects the reference's
    per-token gather loop (:444-466) or an index_select restatement of it.
    """
    num_heads, head_dim = q.shape[1], q.shape[3]
    num_groups = num_heads // k_cache.shape[1]
    gather = gather_kv_cache_loop if literal_gather else gather_kv_cache
    outs = []
    for i in range(q.shape[2]):
        k_full, v_full = gather(int(positions[i]), block_tables[i], k_cache, v_cache)  # :362-367
        q_i = q[:, :, i : i + 1, :]  # :369-371
        k_full = k_full.unsqueeze(0).repeat_interleave(num_groups, dim=1)  # :372-374
        v_full = v_full.unsqueeze(0).repeat_interleave(num_groups, dim=1)  # :375-377
        out_i = F.scaled_dot_product_attention(q_i, k_full, v_full, attn_mask=None, scale=head_dim**-0.5)
        outs.append(out_i)  # :378-385
    out = torch.cat(outs, dim=2)  # :411-413, (1, Hq, B, D)
    return out[0].transpose(0, 1).contiguous()
