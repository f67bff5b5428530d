"""Synthetic workloads: determinism, shapes, and the work formulas (CPU)."""

import math

import torch

from tinyserver_amd import workloads as W


def test_deterministic_and_shaped():
    a = W.make("qwen3-0.6b-decode-bs4")
    b = W.make("qwen3-0.6b-decode-bs4")
    assert torch.equal(a.k_cache, b.k_cache) and torch.equal(a.q, b.q) and a.block_lists == b.block_lists
    assert a.k_cache.shape == (256, 8, 16, 128) and a.q.shape == (4, 16, 128) and a.k.shape == (4, 8, 128)
    assert all(16 <= int(n) <= 512 for n in a.ctx_lens)
    pages = [p for lst in a.block_lists for p in lst]
    assert len(pages) == len(set(pages)), "pages must be disjoint"
    for lst, n in zip(a.block_lists, a.ctx_lens):
        assert len(lst) == math.ceil(int(n) / 16)


def test_prefill_layout():
    p = W.make_prefill("t", 3, 3, 8, 2, 10, 40)
    cu = p.cu_seqlens.tolist()
    assert cu[0] == 0 and cu[-1] == p.q.shape[0] and p.cos.shape == (p.q.shape[0], 128)
    assert torch.equal(p.positions[cu[1] : cu[2]], torch.arange(cu[2] - cu[1]))


def test_poison_marks_unused_slots():
    w = W.make("qwen3-0.6b-decode-bs4", poison=True)
    for lst, n in zip(w.block_lists, w.ctx_lens):
        last = lst[-1]
        used = (int(n) - 1) - (len(lst) - 1) * 16  # slots holding positions < ctx-1 in the last page
        assert (w.k_cache[last, :, used:] == 1e4).all()
        if used > 0:
            assert (w.k_cache[last, :, :used] != 1e4).all()


def test_work_formulas():
    # decode: K+V once per token per kv head, q in / o out, table entries, seq_lens
    assert W.decode_bytes([16, 17], 4, 2, head_dim=128) == (33 * 2 * 128 * 2 * 2) + 2 * 2 * 4 * 128 * 2 + 3 * 4 + 8
    # prefill: 4 D Hq sum L(L+1)/2
    assert W.prefill_flops([1, 3], 2, head_dim=8) == 4 * 8 * 2 * (1 + 6)


def test_mixed_step_shares_one_pool():
    """The continuous-batching step: prefill and decode halves on one pool,
    disjoint pages, the decode prefixes kept and everything else poisoned."""
    m = W.make_mixed("t", 5, decode_batch=6, ctx_lo=20, ctx_hi=90, prefill_seqs=3, len_lo=5, len_hi=40,
                     num_heads=8, num_kv_heads=2, poison=True)
    assert m.prefill.k_cache is m.decode.k_cache and m.prefill.v_cache is m.decode.v_cache
    assert m.prefill.q_weight is m.decode.q_weight and m.prefill.k_weight is m.decode.k_weight
    pages = [p for lst in m.decode.block_lists + m.prefill.block_lists for p in lst]
    assert len(pages) == len(set(pages)), "the halves must own disjoint pages"
    assert m.k_cache.shape[0] == math.ceil(len(pages) * 1.1)
    for lst, n in zip(m.decode.block_lists, m.decode.ctx_lens):
        assert len(lst) == math.ceil(int(n) / 16)
    for i, lst in enumerate(m.prefill.block_lists):
        assert len(lst) == math.ceil(int(m.prefill.seq_lens[i]) / 16)
        assert (m.k_cache[lst] == 1e4).all()  # pages the prefill store will fill
    assert m.decode.block_tables.shape == (6, max(len(l) for l in m.decode.block_lists))
    assert m.prefill.block_tables.shape == (3, max(len(l) for l in m.prefill.block_lists))
    for i, lst in enumerate(m.decode.block_lists):
        assert m.decode.block_tables[i, : len(lst)].tolist() == lst
    assert m.prefill.cu_seqlens[-1] == m.prefill.q.shape[0] and m.decode.q.shape == (6, 8, 128)
    n = W.make_mixed("t", 5, decode_batch=6, ctx_lo=20, ctx_hi=90, prefill_seqs=3, len_lo=5, len_hi=40,
                     num_heads=8, num_kv_heads=2, poison=True)
    assert torch.equal(n.k_cache, m.k_cache) and torch.equal(n.prefill.q, m.prefill.q)
