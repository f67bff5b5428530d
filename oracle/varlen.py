"""Varlen causal prefill, restated on the CPU (test infrastructure).

* ``flash_attn_varlen_func`` -- the Triton kernel's algorithm
  (server/model/kernels/varlen_attention.py:8-142, wrapper :145-218): per
  (sequence, q-head) an fp32 online softmax over 32-key blocks, GQA
  kv head = h // (Hq / Hkv), top-left causal mask q_idx >= k_idx within the
  sequence (:116-119), p cast to the V dtype before P.V (:126) while l sums
  the fp32 p (:128-129), out = acc / l in the query dtype. Every query row of a
  sequence is processed at once; 32-key blocks are walked in ascending order as
  the kernel walks them, so the running max -- and therefore the bf16
  rounding of p -- follows the kernel's sequence.
* ``reference_attn_varlen`` -- the reference's naive check
  (varlen_attention.py:224-254).
* ``prefill_sdpa_block_mask`` -- the reference's CPU prefill branch
  (server/model/patches/qwen3.py:132-171): one SDPA over the packed tokens
  with a block-diagonal causal mask.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

BLOCK_N = 32  # varlen_attention.py:190


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, causal, softmax_scale=None):
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:  # :172-173
        raise ValueError("q, k, v must be 3D tensors")
    _, num_heads_q, head_dim = q.shape
    num_heads_k = k.shape[1]
    if num_heads_q % num_heads_k != 0:  # :178-179
        raise ValueError("num_heads_q must be divisible by num_heads_k for GQA")
    if softmax_scale is None:  # :183-184
        softmax_scale = 1.0 / (head_dim**0.5)
    group = num_heads_q // num_heads_k
    kv_head = torch.arange(num_heads_q) // group  # :42-43
    out = torch.empty_like(q)
    cq = [int(x) for x in cu_seqlens_q.tolist()]
    ck = [int(x) for x in cu_seqlens_k.tolist()]
    for b in range(len(cq) - 1):
        q_start, q_len = cq[b], cq[b + 1] - cq[b]  # :45-58
        k_start, k_len = ck[b], ck[b + 1] - ck[b]
        if q_len <= 0:
            continue
        qs = q[q_start : q_start + q_len].transpose(0, 1).to(torch.float32)  # (Hq, Lq, D)
        ks = k[k_start : k_start + k_len].transpose(0, 1)[kv_head].to(torch.float32)  # (Hq, Lk, D)
        vs = v[k_start : k_start + k_len].transpose(0, 1)[kv_head]  # (Hq, Lk, D), V dtype
        m = torch.full((num_heads_q, q_len), float("-inf"))
        l = torch.zeros((num_heads_q, q_len))
        acc = torch.zeros((num_heads_q, q_len, head_dim))
        rows = torch.arange(q_len)
        # :86-90 -- the last (widest) 32-row query block bounds every other one;
        # blocks beyond a row's own bound are fully masked for it and change nothing.
        end = k_len if not causal else min(k_len, -(-q_len // 32) * 32)
        for kb in range(0, end, BLOCK_N):  # :92
            cols = kb + torch.arange(BLOCK_N)
            inb = cols < k_len  # :99, :115
            kk = torch.zeros((num_heads_q, BLOCK_N, head_dim))
            vv = torch.zeros((num_heads_q, BLOCK_N, head_dim), dtype=v.dtype)
            n = int(inb.sum())
            kk[:, :n] = ks[:, kb : kb + n]
            vv[:, :n] = vs[:, kb : kb + n]
            qk = torch.matmul(qs, kk.transpose(1, 2)) * softmax_scale  # :111-112
            mask = inb[None, :].expand(q_len, BLOCK_N)
            if causal:
                mask = mask & (rows[:, None] >= cols[None, :])  # :116-119
            qk = torch.where(mask[None], qk, float("-inf"))
            m_new = torch.maximum(m, qk.max(-1).values)  # :121
            # A row whose every key so far is masked keeps m = -inf; guard the
            # (-inf) - (-inf) the kernel never reaches for rows it visits.
            safe = torch.isfinite(m_new)
            p = torch.where(safe[..., None], torch.exp(qk - torch.where(safe, m_new, 0.0)[..., None]), 0.0)  # :122
            alpha = torch.where(safe, torch.exp(m - torch.where(safe, m_new, 0.0)), 1.0)  # :123
            acc = acc * alpha[..., None] + torch.matmul(p.to(v.dtype).float(), vv.float())  # :125-126
            l = l * alpha + p.sum(-1)  # :128-129
            m = m_new
        o = acc / l[..., None]  # :132
        out[q_start : q_start + q_len] = o.transpose(0, 1).to(q.dtype)  # :133-142
    return out


def reference_attn_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, causal, sm_scale):
    """_reference_attn_varlen (varlen_attention.py:224-254), bottom-right causal."""
    batch = cu_seqlens_q.shape[0] - 1
    nheads_q, nheads_k = q.shape[1], k.shape[1]
    heads_per_group = nheads_q // nheads_k
    out = torch.zeros_like(q)
    for b in range(batch):
        qs, qe = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
        ks, ke = int(cu_seqlens_k[b]), int(cu_seqlens_k[b + 1])
        sq, sk = qe - qs, ke - ks
        for hq in range(nheads_q):
            hk = hq // heads_per_group
            qi, ki, vi = q[qs:qe, hq], k[ks:ke, hk], v[ks:ke, hk]
            s = (qi @ ki.T) * sm_scale
            if causal:
                offset = sk - sq
                row_idx = torch.arange(sq)[:, None]
                col_idx = torch.arange(sk)[None, :]
                s = s.masked_fill(~((row_idx + offset) >= col_idx), float("-inf"))
            p = torch.softmax(s.float(), dim=-1).to(q.dtype)
            out[qs:qe, hq] = p @ vi
    return out


def prefill_sdpa_block_mask(q, k, v, seq_lens, head_dim):
    """_prefill_sdpa_with_block_mask (server/model/patches/qwen3.py:132-171).

    q: (1, Hq, T, D), k/v: (1, Hkv, T, D). Returns (1, T, Hq*D).
    """
    total = q.shape[2]
    mask = torch.full((total, total), float("-inf"), dtype=q.dtype)
    start = 0
    for n in seq_lens:
        n = int(n)
        mask[start : start + n, start : start + n] = torch.triu(torch.full((n, n), float("-inf"), dtype=q.dtype), diagonal=1)
        start += n
    out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=head_dim**-0.5, enable_gqa=True)
    return out.transpose(1, 2).reshape(1, total, -1)


def prefill_sdpa_per_sequence(q, k, v, cu_seqlens, head_dim=None):
    """The same prefill math as the reference's CPU branch
    (server/model/patches/qwen3.py:132-171: causal SDPA within each sequence,
    GQA), vectorised per sequence instead of one block-diagonal mask over the
    packed tokens: one causal SDPA per sequence, in the inputs' dtype.

    q: (T, Hq, D), k/v: (T, Hkv, D) token-major; returns (T, Hq, D).
    """
    head_dim = head_dim or q.shape[-1]
    out = torch.empty_like(q)
    cu = [int(x) for x in cu_seqlens.tolist()]
    for b in range(len(cu) - 1):
        a, e = cu[b], cu[b + 1]
        if e <= a:
            continue
        qs = q[a:e].transpose(0, 1)[None]  # (1, Hq, L, D)
        ks = k[a:e].transpose(0, 1)[None]
        vs = v[a:e].transpose(0, 1)[None]
        o = F.scaled_dot_product_attention(qs, ks, vs, is_causal=True, scale=head_dim**-0.5, enable_gqa=True)
        out[a:e] = o[0].transpose(0, 1)
    return out
