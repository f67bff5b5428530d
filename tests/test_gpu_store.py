"""Paged K/V store on the GPU vs the oracle: bit-exact.

Cases are the reference's own (tests/model/test_kv_cache_kernels.py:73-207:
batched == per-sequence for a single sequence, three ragged sequences, a
multi-block sequence, one token each and non-zero start positions), plus the
device-side addressing variant at the decode and prefill shapes, int32/int64
mappings, out-of-range ids (skipped, never written) and the full
Qwen3-8B-shaped prefill store checked by gathering every token back.
"""

import pytest
import torch

from oracle import kv_store as ok
from tests.helpers import assert_bitexact
from tinyserver_amd import workloads as W
from tinyserver_amd.kernels import store_kv_cache, store_kv_cache_batched, store_kv_cache_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"

REF_CASES = [
    # (num_kv_heads, block_size, head_dim, num_blocks, seqs) -- test_kv_cache_kernels.py:73-207
    (2, 4, 8, 2, [dict(start_pos=0, seq_len=4, block_table=[0])]),
    (4, 4, 16, 4, [dict(start_pos=0, seq_len=3, block_table=[0]), dict(start_pos=0, seq_len=5, block_table=[1, 2]),
                   dict(start_pos=0, seq_len=4, block_table=[3])]),
    (2, 4, 32, 3, [dict(start_pos=0, seq_len=12, block_table=[0, 1, 2])]),
    (2, 4, 8, 3, [dict(start_pos=0, seq_len=1, block_table=[b]) for b in range(3)]),
    (2, 4, 8, 3, [dict(start_pos=4, seq_len=3, block_table=[0, 1]), dict(start_pos=8, seq_len=4, block_table=[0, 0, 2])]),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", range(len(REF_CASES)))
def test_reference_cases(case, dtype):
    hkv, bs, d, nb, seqs = REF_CASES[case]
    g = torch.Generator().manual_seed(case)
    ks = [torch.randn(hkv, s["seq_len"], d, generator=g).to(dtype) for s in seqs]
    vs = [torch.randn(hkv, s["seq_len"], d, generator=g).to(dtype) for s in seqs]
    shape = (nb, hkv, bs, d)
    # oracle, per sequence
    kr, vr = torch.zeros(shape, dtype=dtype), torch.zeros(shape, dtype=dtype)
    for s, k, v in zip(seqs, ks, vs):
        ok.store_kv_cache(s["start_pos"], torch.tensor(s["block_table"]), k, v, kr, vr)
    # GPU per sequence
    kp, vp = torch.zeros(shape, dtype=dtype, device=DEV), torch.zeros(shape, dtype=dtype, device=DEV)
    for s, k, v in zip(seqs, ks, vs):
        bt = torch.tensor(s["block_table"], dtype=torch.int32, device=DEV)
        store_kv_cache(s["start_pos"], bt, k.to(DEV), v.to(DEV), kp, vp)
    # GPU batched through the reference's mapping rule (test_kv_cache_kernels.py:16-37)
    bm, sm = [], []
    for s in seqs:
        for i in range(s["seq_len"]):
            p = s["start_pos"] + i
            bm.append(s["block_table"][p // bs])
            sm.append(p % bs)
    kb, vb = torch.zeros(shape, dtype=dtype, device=DEV), torch.zeros(shape, dtype=dtype, device=DEV)
    store_kv_cache_batched(torch.cat(ks, 1).to(DEV), torch.cat(vs, 1).to(DEV), kb, vb,
                           torch.tensor(bm, dtype=torch.int32, device=DEV), torch.tensor(sm, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    for name, got in (("per-seq K", kp), ("per-seq V", vp), ("batched K", kb), ("batched V", vb)):
        assert_bitexact(got, kr if "K" in name else vr, name)


@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_mapped_matches_oracle_prefill_shape(index_dtype):
    w = W.make("qwen3-4b-prefill-8seq")
    blocks, slots = ok.build_block_slot_mappings(
        [{"num_tokens": int(n), "block_table": b} for n, b in zip(w.seq_lens, w.block_lists)], W.PAGE)
    k_src, v_src = w.k.transpose(0, 1).contiguous(), w.v.transpose(0, 1).contiguous()
    kr, vr = w.k_cache.clone(), w.v_cache.clone()
    ok.store_kv_cache_batched(k_src, v_src, kr, vr, blocks, slots)
    kc, vc = w.k_cache.to(DEV), w.v_cache.to(DEV)
    store_kv_cache_batched(k_src.to(DEV), v_src.to(DEV), kc, vc, blocks.to(index_dtype).to(DEV),
                           slots.to(index_dtype).to(DEV))
    torch.cuda.synchronize()
    assert_bitexact(kc, kr, "K")
    assert_bitexact(vc, vr, "V")


def test_paged_prefill_matches_mapped():
    """Device-side addressing == the call site's mapping loop (qwen3.py:296-318)."""
    w = W.make("qwen3-4b-prefill-8seq")
    blocks, slots = ok.build_block_slot_mappings(
        [{"num_tokens": int(n), "block_table": b} for n, b in zip(w.seq_lens, w.block_lists)], W.PAGE)
    kr, vr = w.k_cache.clone(), w.v_cache.clone()
    ok.store_kv_cache_batched(w.k.transpose(0, 1), w.v.transpose(0, 1), kr, vr, blocks, slots)
    kc, vc = w.k_cache.to(DEV), w.v_cache.to(DEV)
    kd, vd = w.k.to(DEV), w.v.to(DEV)
    # (T, Hkv, D) projections passed as (Hkv, T, D) views, no copy.
    store_kv_cache_paged(kd.transpose(0, 1), vd.transpose(0, 1), kc, vc, w.block_tables.to(DEV),
                         w.cu_seqlens.to(DEV))
    torch.cuda.synchronize()
    assert_bitexact(kc, kr, "K")
    assert_bitexact(vc, vr, "V")


@pytest.mark.parametrize("pos_dtype", [torch.int32, torch.int64])
def test_paged_decode_positions(pos_dtype):
    """One token per sequence at position ctx-1 (the decode loop, qwen3.py:335-357)."""
    w = W.make("qwen3-0.6b-decode-bs4", poison=True)
    kr, vr = w.k_cache.clone(), w.v_cache.clone()
    for i in range(len(w.ctx_lens)):
        ok.store_kv_cache(int(w.positions[i]), torch.tensor(w.block_lists[i]), w.k[i][:, None], w.v[i][:, None], kr, vr)
    kc, vc = w.k_cache.to(DEV), w.v_cache.to(DEV)
    b = len(w.ctx_lens)
    cu = torch.arange(b + 1, dtype=torch.int32, device=DEV)
    store_kv_cache_paged(w.k.to(DEV).transpose(0, 1), w.v.to(DEV).transpose(0, 1), kc, vc, w.block_tables.to(DEV), cu,
                         w.positions.to(pos_dtype).to(DEV))
    torch.cuda.synchronize()
    assert_bitexact(kc, kr, "K")
    assert_bitexact(vc, vr, "V")


def test_out_of_range_ids_are_skipped():
    hkv, bs, d, nb = 2, 16, 128, 4
    src = torch.randn(hkv, 3, d, device=DEV).to(torch.bfloat16)
    kc = torch.zeros(nb, hkv, bs, d, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    bm = torch.tensor([1, nb, -1], dtype=torch.int64, device=DEV)  # only token 0 is in range
    sm = torch.tensor([2, 0, 0], dtype=torch.int64, device=DEV)
    store_kv_cache_batched(src, src, kc, vc, bm, sm)
    # A position past the block table is skipped too.
    store_kv_cache(40, torch.tensor([0, 1], dtype=torch.int32, device=DEV), src[:, :1], src[:, :1], kc, vc)
    torch.cuda.synchronize()
    expect = torch.zeros(nb, hkv, bs, d, dtype=torch.bfloat16)
    expect[1, :, 2] = src[:, 0].cpu()
    assert_bitexact(kc, expect, "K")


def test_full_prefill_store_roundtrip():
    """Qwen3-8B prefill shape, every token: gather back == source (bit-exact)."""
    w = W.make("qwen3-8b-prefill-16seq", device=DEV)
    kc, vc = w.k_cache.clone(), w.v_cache.clone()
    store_kv_cache_paged(w.k.transpose(0, 1), w.v.transpose(0, 1), kc, vc, w.block_tables, w.cu_seqlens)
    torch.cuda.synchronize()
    cu = w.cu_seqlens.tolist()
    for s, lst in enumerate(w.block_lists):
        n = cu[s + 1] - cu[s]
        pos = torch.arange(n, device=DEV)
        blocks = torch.tensor(lst, device=DEV)[pos // W.PAGE]
        got_k = kc[blocks, :, pos % W.PAGE, :]  # (n, Hkv, D)
        got_v = vc[blocks, :, pos % W.PAGE, :]
        assert torch.equal(got_k, w.k[cu[s]:cu[s + 1]]), f"seq {s} K"
        assert torch.equal(got_v, w.v[cu[s]:cu[s + 1]]), f"seq {s} V"
