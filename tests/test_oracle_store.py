"""Pins for the oracle's paged K/V store (CPU).

* The reference's own cases (tests/model/test_kv_cache_kernels.py:73-207):
  batched store == per-sequence store for one sequence, three ragged
  sequences, a multi-block sequence, one token each, non-zero start positions.
* A brute-force per-element loop of the address rule
  cache[bt[p // BS], h, p % BS, d] = src[h, t, d] on tiny inputs.
* The inverse: gather_kv_cache (server/model/patches/qwen3.py:423-466) reads
  back exactly what was stored, for the vectorised and the per-token gather.
* The prefill mapping rule (qwen3.py:296-303) against a hand-written table.
* The reference's ValueError guards (test_kv_cache_kernels.py:210-255).
"""

import pytest
import torch

from oracle import kv_store as ok

REF_CASES = [
    (2, 4, 8, 2, [dict(start_pos=0, seq_len=4, block_table=[0])]),
    (4, 4, 16, 4, [dict(start_pos=0, seq_len=3, block_table=[0]), dict(start_pos=0, seq_len=5, block_table=[1, 2]),
                   dict(start_pos=0, seq_len=4, block_table=[3])]),
    (2, 4, 32, 3, [dict(start_pos=0, seq_len=12, block_table=[0, 1, 2])]),
    (2, 4, 8, 3, [dict(start_pos=0, seq_len=1, block_table=[b]) for b in range(3)]),
    (2, 4, 8, 3, [dict(start_pos=4, seq_len=3, block_table=[0, 1]), dict(start_pos=8, seq_len=4, block_table=[0, 0, 2])]),
]


def _brute(seqs, srcs, shape):
    cache = torch.zeros(shape)
    hkv, bs, d = shape[1], shape[2], shape[3]
    for s, src in zip(seqs, srcs):
        for t in range(s["seq_len"]):
            p = s["start_pos"] + t
            for h in range(hkv):
                for e in range(d):
                    cache[s["block_table"][p // bs], h, p % bs, e] = src[h, t, e]
    return cache


@pytest.mark.parametrize("case", range(len(REF_CASES)))
def test_reference_cases(case):
    hkv, bs, d, nb, seqs = REF_CASES[case]
    g = torch.Generator().manual_seed(case)
    ks = [torch.randn(hkv, s["seq_len"], d, generator=g) for s in seqs]
    vs = [torch.randn(hkv, s["seq_len"], d, generator=g) for s in seqs]
    shape = (nb, hkv, bs, d)
    kp, vp = torch.zeros(shape), torch.zeros(shape)
    for s, k, v in zip(seqs, ks, vs):
        ok.store_kv_cache(s["start_pos"], torch.tensor(s["block_table"], dtype=torch.int32), k, v, kp, vp)
    bm, sm = ok.build_block_slot_mappings(
        [{"num_tokens": s["seq_len"], "block_table": s["block_table"]} for s in seqs], bs,
        start_positions=[s["start_pos"] for s in seqs])
    kb, vb = torch.zeros(shape), torch.zeros(shape)
    ok.store_kv_cache_batched(torch.cat(ks, 1), torch.cat(vs, 1), kb, vb, bm, sm)
    assert torch.equal(kb, kp) and torch.equal(vb, vp)
    assert torch.equal(kp, _brute(seqs, ks, shape)) and torch.equal(vp, _brute(seqs, vs, shape))


def test_gather_is_the_inverse():
    g = torch.Generator().manual_seed(7)
    hkv, bs, d, n = 4, 16, 128, 77
    nb = 12
    table = torch.randperm(nb, generator=g)[: (n + bs - 1) // bs].tolist()
    k = torch.randn(hkv, n, d, generator=g).to(torch.bfloat16)
    v = torch.randn(hkv, n, d, generator=g).to(torch.bfloat16)
    kc = torch.full((nb, hkv, bs, d), 1e4, dtype=torch.bfloat16)
    vc = kc.clone()
    ok.store_kv_cache(0, torch.tensor(table), k, v, kc, vc)
    for gather in (ok.gather_kv_cache, ok.gather_kv_cache_loop):
        kf, vf = gather(n - 1, table, kc, vc)
        assert torch.equal(kf, k) and torch.equal(vf, v)


def test_prefill_mapping_rule():
    seqs = [{"num_tokens": 3, "block_table": [7]}, {"num_tokens": 6, "block_table": [2, 5]}]
    bm, sm = ok.build_block_slot_mappings(seqs, 4)
    assert bm.tolist() == [7, 7, 7, 2, 2, 2, 2, 5, 5]
    assert sm.tolist() == [0, 1, 2, 0, 1, 2, 3, 0, 1]


def test_guards():
    kc = torch.zeros(2, 2, 4, 8)
    with pytest.raises(ValueError, match="3D"):
        ok.store_kv_cache_batched(torch.zeros(2, 8), torch.zeros(2, 1, 8), kc, kc.clone(), torch.zeros(1),
                                  torch.zeros(1))
    with pytest.raises(ValueError):
        ok.store_kv_cache_batched(torch.zeros(2, 3, 8), torch.zeros(2, 4, 8), kc, kc.clone(), torch.zeros(3),
                                  torch.zeros(3))
    with pytest.raises(ValueError):
        ok.store_kv_cache_batched(torch.zeros(2, 4, 8), torch.zeros(2, 4, 8), kc, kc.clone(), torch.zeros(3),
                                  torch.zeros(4))
    with pytest.raises(ValueError, match="3D"):
        ok.store_kv_cache(0, torch.zeros(1, dtype=torch.int32), torch.zeros(2, 8), torch.zeros(2, 1, 8), kc,
                          kc.clone())
