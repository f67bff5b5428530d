"""Paged decode attention on the GPU vs the oracle.

The oracle restates the reference kernel (paged_attention.py:8-121) in fp32.
Cases: the reference's own three configurations, query not mutated, shape and
dtype, the poisoned partial last block (tests/model/test_paged_attention_kernel.py:
109-222); the Qwen3-0.6B-shaped decode step end to end (norm+RoPE+store then
attend); GQA groups 1..16, head_dim 64/128, page sizes 4..64; small batches in
one workgroup per (sequence, kv head) unit (no merge launch); split-K with
forced small splits, called twice to show the merge counters reset; seq_len 1
(output = the V row); the full Qwen3-8B bs64 and Qwen3-32B bs32 batches, every sequence and
head. Tolerance for bf16/fp16: max-abs 2e-2, mean-abs 2e-3;
fp32 (generic kernel): the reference test's 1e-3.
"""

import math

import pytest
import torch

from oracle import kv_store as ok
from oracle import norm_rope as onr
from oracle import paged as op
from tests.helpers import assert_close
from tinyserver_amd import workloads as W
from tinyserver_amd.kernels import paged_attention_forward, paged_decode_step, qk_norm_rope_store

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _random_paged_inputs(seq_lens, num_heads, num_kv_heads, head_dim, block_size, dtype, seed):
    """The reference test's generator (test_paged_attention_kernel.py:67-106): disjoint
    shuffled physical blocks plus 3 spare ones, zero-padded tables."""
    gen = torch.Generator().manual_seed(seed)
    blocks_per_seq = [max(1, math.ceil(n / block_size)) for n in seq_lens]
    num_blocks = sum(blocks_per_seq) + 3

    def randn(*shape):
        return torch.randn(*shape, generator=gen).to(dtype)

    query = randn(len(seq_lens), num_heads, head_dim)
    k_cache = randn(num_blocks, num_kv_heads, block_size, head_dim)
    v_cache = randn(num_blocks, num_kv_heads, block_size, head_dim)
    phys = torch.randperm(num_blocks, generator=gen)[: sum(blocks_per_seq)]
    bt = torch.zeros(len(seq_lens), max(blocks_per_seq), dtype=torch.int32)
    cur = 0
    for s, n in enumerate(blocks_per_seq):
        bt[s, :n] = phys[cur : cur + n].to(torch.int32)
        cur += n
    return query, k_cache, v_cache, bt, torch.tensor(seq_lens, dtype=torch.int32)


def _run(query, k_cache, v_cache, bt, bs, sl, **kw):
    out = paged_attention_forward(query.to(DEV), k_cache.to(DEV), v_cache.to(DEV), bt.to(DEV), bs, sl.to(DEV), **kw)
    torch.cuda.synchronize()
    return out


REF_CONFIGS = [
    (4, 4, 64, 16, [10]),
    (8, 2, 64, 16, [7, 16, 40]),
    (16, 4, 128, 32, [1, 33, 64]),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cfg", range(len(REF_CONFIGS)))
def test_reference_configs(cfg, dtype):
    hq, hkv, d, bs, lens = REF_CONFIGS[cfg]
    args = _random_paged_inputs(lens, hq, hkv, d, bs, dtype, seed=0)
    out = _run(*args[:4], bs, args[4])
    ref = op.paged_attention_forward(*args[:4], bs, args[4])
    tol = dict(max_abs=1e-3, mean_abs=1e-3) if dtype == torch.float32 else {}
    assert out.dtype == dtype and out.shape == args[0].shape
    assert_close(out, ref, what=f"cfg{cfg} {dtype}", **tol)


def test_query_not_mutated():
    q, kc, vc, bt, sl = _random_paged_inputs([12, 5], 8, 2, 64, 16, torch.bfloat16, seed=1)
    qd = q.to(DEV)
    before = qd.clone()
    paged_attention_forward(qd, kc.to(DEV), vc.to(DEV), bt.to(DEV), 16, sl.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(qd, before)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_partial_last_block_masked(dtype):
    q, kc, vc, bt, sl = _random_paged_inputs([5], 8, 2, 64, 16, dtype, seed=3)
    blk = int(bt[0, 0])
    kc[blk, :, 5:, :] = 1e4
    vc[blk, :, 5:, :] = 1e4
    out = _run(q, kc, vc, bt, 16, sl)
    ref = op.paged_attention_forward(q, kc, vc, bt, 16, sl)
    tol = dict(max_abs=1e-3, mean_abs=1e-3) if dtype == torch.float32 else {}
    assert_close(out, ref, what="poison", **tol)


def test_nonfinite_unused_slots_do_not_leak():
    q, kc, vc, bt, sl = _random_paged_inputs([21], 8, 2, 128, 16, torch.bfloat16, seed=4)
    blk = int(bt[0, 1])
    kc[blk, :, 5:, :] = float("nan")
    vc[blk, :, 5:, :] = float("inf")
    out = _run(q, kc, vc, bt, 16, sl)
    ref = op.paged_attention_forward(q, kc, vc, bt, 16, sl)
    assert_close(out, ref, what="nan/inf slots")


@pytest.mark.parametrize("group", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_gqa_groups(group, head_dim):
    hkv = 2
    q, kc, vc, bt, sl = _random_paged_inputs([1, 17, 300, 64], hkv * group, hkv, head_dim, 16, torch.bfloat16,
                                             seed=group)
    out = _run(q, kc, vc, bt, 16, sl)
    ref = op.paged_attention_forward(q, kc, vc, bt, 16, sl)
    assert_close(out, ref, what=f"G={group} D={head_dim}")


@pytest.mark.parametrize("block_size", [4, 8, 32, 64, 128, 256])
def test_page_sizes(block_size):
    """Page sizes up to the server's default of 256 tokens."""
    q, kc, vc, bt, sl = _random_paged_inputs([3, 50, 129, 16], 16, 4, 128, block_size, torch.bfloat16, seed=7)
    out = _run(q, kc, vc, bt, block_size, sl)
    ref = op.paged_attention_forward(q, kc, vc, bt, block_size, sl)
    assert_close(out, ref, what=f"BS={block_size}")


@pytest.mark.parametrize("num_workgroups", [1, 3, 7, 64, 333, 4096])
def test_stream_partition(num_workgroups):
    """Sequences cut between workgroups at every kind of boundary (one workgroup,
    a few, more workgroups than tiles); a second call reuses the workspace."""
    q, kc, vc, bt, sl = _random_paged_inputs([2000, 1, 777, 4096, 64, 0, 16], 32, 8, 128, 16, torch.bfloat16,
                                             seed=9)
    ref = op.paged_attention_forward(q, kc, vc, bt, 16, sl)
    for call in range(2):
        out = _run(q, kc, vc, bt, 16, sl, num_workgroups=num_workgroups).cpu()
        assert torch.isnan(out[5]).all(), "empty sequence must give NaN (0/0) like the reference"
        keep = [0, 1, 2, 3, 4, 6]
        assert_close(out[keep], ref[keep], what=f"W={num_workgroups} call {call}")


UNIT_CASES = [
    # (num_heads, num_kv_heads, head_dim, block_size, dtype, seq_lens)
    (16, 8, 128, 16, torch.bfloat16, [0, 1, 5, 63, 300, 512]),
    (32, 8, 128, 16, torch.float16, [17, 512, 2, 33]),
    (8, 8, 64, 16, torch.bfloat16, [3, 64, 511, 100, 1, 16, 250]),
    (64, 4, 128, 32, torch.bfloat16, [500, 31, 1, 96]),
    (16, 4, 128, 8, torch.bfloat16, [7, 512, 130]),
]


@pytest.mark.parametrize("case", range(len(UNIT_CASES)))
def test_unit_form(case):
    """With no grid asked for, a batch of at most 64 (sequence, kv head) units
    whose block tables hold at most 512 tokens runs one workgroup per unit:
    its four waves split the unit's tiles (some waves get none when a unit
    has fewer than four tiles) and merge in LDS, with no merge launch. Every
    such case here -- an empty sequence (NaN), seq_len 1, a full 512-token
    table, head_dim 64, groups of 1 to 16 heads, 8-, 16- and 32-token pages,
    bf16 and f16 -- against the oracle, and against the stream form that an
    explicit grid takes."""
    hq, hkv, d, bs, dtype, lens = UNIT_CASES[case]
    q, kc, vc, bt, sl = _random_paged_inputs(lens, hq, hkv, d, bs, dtype, seed=60 + case)
    assert len(lens) * hkv <= 64 and bt.shape[1] * bs <= 512
    print(f"unit form: heads {hq}/{hkv}, head_dim {d}, page {bs}, {dtype}, lens {lens}", flush=True)
    ref = op.paged_attention_forward(q, kc, vc, bt, bs, sl)
    out = _run(q, kc, vc, bt, bs, sl).cpu()
    stream = _run(q, kc, vc, bt, bs, sl, num_workgroups=16).cpu()
    keep = [i for i, n in enumerate(lens) if n > 0]
    for i, n in enumerate(lens):
        if n == 0:
            assert torch.isnan(out[i]).all(), "empty sequence must give NaN (0/0) like the reference"
    assert_close(out[keep], ref[keep], what=f"unit form case {case}")
    assert_close(out[keep], stream[keep], what=f"unit form vs stream form, case {case}")


def test_workspace_reuse_across_shapes():
    """Calls of different shapes and worker counts alternating on one
    workspace: nothing a call leaves in it (partials over a wide range from a
    small call with many workers) can disturb a later call."""
    big = _random_paged_inputs([3000, 17, 900, 64, 2500, 1, 4000, 333], 32, 8, 128, 16, torch.bfloat16, seed=41)
    small = _random_paged_inputs([700, 5], 16, 4, 128, 16, torch.bfloat16, seed=42)
    refs = [op.paged_attention_forward(*x[:4], 16, x[4]) for x in (big, small)]
    for call, (x, ref, nwg) in enumerate([(big, refs[0], 0), (small, refs[1], 4096), (big, refs[0], 7),
                                          (small, refs[1], 1), (big, refs[0], 0)]):
        out = _run(*x[:4], 16, x[4], num_workgroups=nwg).cpu()
        assert_close(out, ref, what=f"call {call} (num_workgroups={nwg})")


def test_repeated_calls_are_identical():
    """More calls than the stream kernel's work-queue slots, two shapes
    interleaved: whichever wave streams a chunk, its partial lands in the same
    slot and the merge order is fixed, so every output is bit-identical."""
    qa, kca, vca, bta, sla = _random_paged_inputs([3000, 17, 900, 64], 32, 8, 128, 16, torch.bfloat16, seed=31)
    qb, kcb, vcb, btb, slb = _random_paged_inputs([257, 1200], 16, 4, 128, 16, torch.bfloat16, seed=32)
    a = [t.to(DEV) for t in (qa, kca, vca, bta)] + [sla.to(DEV)]
    b = [t.to(DEV) for t in (qb, kcb, vcb, btb)] + [slb.to(DEV)]
    first_a = paged_attention_forward(a[0], a[1], a[2], a[3], 16, a[4])
    first_b = paged_attention_forward(b[0], b[1], b[2], b[3], 16, b[4])
    for _ in range(40):
        oa = paged_attention_forward(a[0], a[1], a[2], a[3], 16, a[4])
        ob = paged_attention_forward(b[0], b[1], b[2], b[3], 16, b[4])
        assert torch.equal(oa, first_a) and torch.equal(ob, first_b)
    assert_close(first_a.cpu(), op.paged_attention_forward(qa, kca, vca, bta, 16, sla), what="repeated calls")


def test_seq_len_one_returns_v_row():
    q, kc, vc, bt, sl = _random_paged_inputs([1, 1], 8, 2, 128, 16, torch.bfloat16, seed=5)
    out = _run(q, kc, vc, bt, 16, sl).cpu()
    for s in range(2):
        for h in range(8):
            assert torch.equal(out[s, h], vc[int(bt[s, 0]), h // 4, 0]), (s, h)


def test_decode_step_qwen3_0p6b():
    """Norm+RoPE+store, then attend (the decode branch, qwen3.py:328-409), vs the oracle."""
    w = W.make("qwen3-0.6b-decode-bs4", poison=True)
    b = len(w.ctx_lens)
    # oracle
    qr, kr = onr.qk_norm_rope(w.q[None], w.k[None], w.q_weight, w.k_weight, w.cos[None], w.sin[None], w.eps)
    kc_ref, vc_ref = w.k_cache.clone(), w.v_cache.clone()
    for i in range(b):
        ok.store_kv_cache(int(w.positions[i]), torch.tensor(w.block_lists[i]), kr[0][:, i : i + 1],
                          w.v[i][:, None], kc_ref, vc_ref)
    ref = op.paged_attention_forward(qr[0].transpose(0, 1).contiguous(), kc_ref, vc_ref, w.block_tables, 16,
                                     w.ctx_lens.to(torch.int32))
    # GPU
    g = w.to(DEV)
    qg, _ = qk_norm_rope_store(g.q, g.k, g.v, g.q_weight, g.k_weight, g.cos, g.sin, g.eps, g.k_cache, g.v_cache,
                               g.block_tables, torch.arange(b + 1, dtype=torch.int32, device=DEV), g.positions,
                               return_k=False)
    out = paged_attention_forward(qg, g.k_cache, g.v_cache, g.block_tables, 16, g.ctx_lens.to(torch.int32))
    torch.cuda.synchronize()
    assert_close(out, ref, what="decode step")


def _full_check(w, num_workgroups=0):
    """w lives on the GPU: every sequence and every head against the oracle
    over the whole pool."""
    out = paged_attention_forward(w.q, w.k_cache, w.v_cache, w.block_tables, 16, w.ctx_lens.to(torch.int32).to(DEV),
                                  num_workgroups=num_workgroups)
    torch.cuda.synchronize()
    out = out.cpu()
    q, kc, vc, bt = w.q.cpu(), w.k_cache.cpu(), w.v_cache.cpu(), w.block_tables.cpu()
    sl = w.ctx_lens.to(torch.int32).cpu()
    print(f"{w.name}: {len(sl)} sequences, ctx {int(sl.min())}..{int(sl.max())}, oracle on the CPU", flush=True)
    ref = op.paged_attention_forward(q, kc, vc, bt, 16, sl)
    assert_close(out, ref, what=f"{w.name}, all {len(sl)} sequences x {q.shape[1]} heads")


def test_qwen3_8b_bs64_full():
    _full_check(W.make("qwen3-8b-decode-bs64", device=DEV))


def test_qwen3_32b_bs32_full():
    _full_check(W.make("qwen3-32b-decode-bs32", device=DEV))


def test_many_sequences():
    """A 1000-sequence decode batch of 1-300 tokens (many small units) against the oracle."""
    g = torch.Generator().manual_seed(45)
    lens = torch.randint(1, 301, (1000,), generator=g).tolist()
    q, kc, vc, bt, sl = _random_paged_inputs(lens, 32, 8, 128, 16, torch.bfloat16, seed=46)
    out = _run(q, kc, vc, bt, 16, sl).cpu()
    ref = op.paged_attention_forward(q, kc, vc, bt, 16, sl)
    assert_close(out, ref, what="1000 sequences")


@pytest.mark.parametrize("batch", [4095, 4096, 12000])
def test_any_batch_size(batch):
    """Batches on both sides of the per-wave LDS tile-prefix limit (4095
    sequences); larger ones read the prefix from the workspace. 1-40 tokens
    per sequence, GQA 2, against the oracle."""
    g = torch.Generator().manual_seed(47 + batch)
    lens = torch.randint(1, 41, (batch,), generator=g).tolist()
    q, kc, vc, bt, sl = _random_paged_inputs(lens, 4, 2, 128, 16, torch.bfloat16, seed=48)
    out = _run(q, kc, vc, bt, 16, sl).cpu()
    ref = op.paged_attention_forward(q, kc, vc, bt, 16, sl)
    assert_close(out, ref, what=f"{batch} sequences")


@pytest.mark.parametrize("name", ["qwen3-0.6b-decode-bs4", "qwen3-8b-decode-bs64"])
def test_fused_decode_step(name):
    """paged_decode_step (norm/RoPE + store + attention, fused) against the
    two-launch path (qk_norm_rope_store, then paged_attention_forward): the
    same rounding and the same operands, so the cache and the output are
    bit-identical; and the output against the oracle."""
    w = W.make(name, poison=True)
    b = len(w.ctx_lens)
    g = w.to(DEV)
    sl = g.ctx_lens.to(torch.int32)
    kc_a, vc_a = g.k_cache.clone(), g.v_cache.clone()
    cu = torch.arange(b + 1, dtype=torch.int32, device=DEV)
    qa, _ = qk_norm_rope_store(g.q, g.k, g.v, g.q_weight, g.k_weight, g.cos, g.sin, g.eps, kc_a, vc_a,
                               g.block_tables, cu, g.positions, return_k=False)
    out_a = paged_attention_forward(qa, kc_a, vc_a, g.block_tables, 16, sl)
    kc_b, vc_b = g.k_cache.clone(), g.v_cache.clone()
    out_b = paged_decode_step(g.q, g.k, g.v, g.q_weight, g.k_weight, g.cos, g.sin, g.eps, kc_b, vc_b,
                              g.block_tables, sl)
    torch.cuda.synchronize()
    assert torch.equal(kc_b, kc_a) and torch.equal(vc_b, vc_a), "cache differs from the two-launch path"
    assert torch.equal(out_b, out_a), "output differs from the two-launch path"
    if b <= 8:  # the oracle on the small batch
        qr, kr = onr.qk_norm_rope(w.q[None], w.k[None], w.q_weight, w.k_weight, w.cos[None], w.sin[None], w.eps)
        kc, vc = w.k_cache.clone(), w.v_cache.clone()
        for i in range(b):
            ok.store_kv_cache(int(w.positions[i]), torch.tensor(w.block_lists[i]), kr[0][:, i : i + 1],
                              w.v[i][:, None], kc, vc)
        ref = op.paged_attention_forward(qr[0].transpose(0, 1).contiguous(), kc, vc, w.block_tables, 16,
                                         w.ctx_lens.to(torch.int32))
        assert_close(out_b, ref, what=f"{name} fused step")


@pytest.mark.parametrize("name", ["qwen3-0.6b-decode-bs4", "qwen3-8b-decode-bs64"])
def test_decode_graph_replays(name):
    """The decode step captured in a HIP graph, as a serving loop replays it:
    the two-launch block (norm/RoPE/store, then attention) and the single-
    launch step, each replayed three times onto freshly poisoned caches with
    eager work between replays, equal to the eager calls in the output and
    both caches."""
    w = W.make(name, poison=True)
    b = len(w.ctx_lens)
    g = w.to(DEV)
    sl = g.ctx_lens.to(torch.int32)
    cu = torch.arange(b + 1, dtype=torch.int32, device=DEV)
    kc_e, vc_e = g.k_cache.clone(), g.v_cache.clone()
    qe, _ = qk_norm_rope_store(g.q, g.k, g.v, g.q_weight, g.k_weight, g.cos, g.sin, g.eps, kc_e, vc_e,
                               g.block_tables, cu, g.positions, return_k=False)
    out_e = paged_attention_forward(qe, kc_e, vc_e, g.block_tables, 16, sl)
    kc, vc = g.k_cache.clone(), g.v_cache.clone()
    q_out = torch.empty_like(qe)
    out_a, out_f = torch.empty_like(out_e), torch.empty_like(out_e)

    def block():
        qk_norm_rope_store(g.q, g.k, g.v, g.q_weight, g.k_weight, g.cos, g.sin, g.eps, kc, vc, g.block_tables, cu,
                           g.positions, q_out=q_out, return_k=False)
        paged_attention_forward(q_out, kc, vc, g.block_tables, 16, sl, out=out_a)

    def step():
        paged_decode_step(g.q, g.k, g.v, g.q_weight, g.k_weight, g.cos, g.sin, g.eps, kc, vc, g.block_tables, sl,
                          out=out_f)

    for fn, out in ((block, out_a), (step, out_f)):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        for rep in range(3):
            kc.copy_(g.k_cache)
            vc.copy_(g.v_cache)
            out.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(kc, kc_e) and torch.equal(vc, vc_e), (fn.__name__, rep, "cache")
            assert torch.equal(out, out_e), (fn.__name__, rep, "output")
            paged_attention_forward(qe, kc_e, vc_e, g.block_tables, 16, sl)  # eager work between replays
            torch.cuda.synchronize()
        del graph


@pytest.mark.parametrize("group,block_size", [(8, 32), (1, 16), (4, 64)])
def test_fused_decode_step_shapes(group, block_size):
    """The single-launch step on GQA groups 8 (two norm passes per unit) and 1
    and on 32- and 64-token pages, with a sequence whose only token is the new
    one: cache and output bit-identical to the two-launch path."""
    gen = torch.Generator().manual_seed(40 + group)
    hkv, d = 2, 128
    hq = group * hkv
    ctx = [1, 17, 300, 1024, 64]
    b = len(ctx)
    q, kc, vc, bt, sl = _random_paged_inputs(ctx, hq, hkv, d, block_size, torch.bfloat16, seed=50 + group)
    k = torch.randn(b, hkv, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(b, hkv, d, generator=gen).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(d, generator=gen)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(d, generator=gen)).to(torch.bfloat16)
    pos = torch.tensor(ctx) - 1
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    emb = torch.cat([pos[:, None].float() * inv, pos[:, None].float() * inv], dim=-1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    t = [x.to(DEV) for x in (q, k, v, qw, kw, cos, sin, bt)]
    slg = sl.to(DEV)
    kc_a, vc_a = kc.to(DEV), vc.to(DEV)
    cu = torch.arange(b + 1, dtype=torch.int32, device=DEV)
    qa, _ = qk_norm_rope_store(t[0], t[1], t[2], t[3], t[4], t[5], t[6], 1e-6, kc_a, vc_a, t[7], cu,
                               pos.to(DEV, torch.int32), return_k=False)
    out_a = paged_attention_forward(qa, kc_a, vc_a, t[7], block_size, slg)
    kc_b, vc_b = kc.to(DEV), vc.to(DEV)
    out_b = paged_decode_step(t[0], t[1], t[2], t[3], t[4], t[5], t[6], 1e-6, kc_b, vc_b, t[7], slg)
    torch.cuda.synchronize()
    assert torch.equal(kc_b, kc_a) and torch.equal(vc_b, vc_a), "cache differs from the two-launch path"
    assert torch.equal(out_b, out_a), "output differs from the two-launch path"
