"""The Qwen3-4B continuous-batching step on one shared KV pool, vs the oracle.

One page-16 pool holds 120 running decode sequences (ctx U[256, 8192]) and
8 new prefill sequences (L U[256, 1024]). The step runs as the scheduler
issues it (server/executor/scheduler.py:128-227): the prefill batch's
forward -- fused QK norm/RoPE + paged store of every token, then varlen
causal attention (server/model/patches/qwen3.py:291-327) -- and then the
decode batch's -- norm/RoPE + store of each new token, then paged decode
attention (:328-416) -- all on one stream, the second reading the pool the
first wrote.

Checked, for every sequence and every head:
* the rotated q and k of both halves against the norm/RoPE oracle (the norm
  tests' bar: at most 1 in 10^4 elements one bf16 ulp off);
* both caches after both halves, bit-exact: the oracle store applied to the
  kernel's own rotated K and the raw V (the store is exact given the same
  rotated K/V), with every slot the step must not touch -- free pages,
  unused tails -- still holding the 1e4 poison;
* all 8 prefill outputs and all 120 decode outputs against the oracle
  attention on the oracle's own rotated q/k (max-abs 2e-2, mean-abs 2e-3).

The same step as an engine batching both would issue it -- one norm/RoPE/
store over the tokens of both batches, then both attentions in one launch
(``mixed_attention``) -- gives every output, the rotated q/k and both caches
bit-identical to the scheduler-order step above (the prefill output within
one bf16 ulp where the scheduler-order step's prefill takes
varlen_prefill_w64, which sums in another order than the one launch's
varlen_prefill_gqa body), and passes the oracle checks too; small cases cover the two-launch fallback (2 q-heads per kv
head) and prefill workgroup counts below and above what is resident.
"""

import pytest
import torch

from oracle import kv_store as ok
from oracle import norm_rope as onr
from oracle import paged as op
from oracle import varlen as ov
from tests.helpers import assert_bitexact, assert_close, assert_within_ulps
from tinyserver_amd import workloads as W
from tinyserver_amd.kernels import flash_attn_varlen_func, mixed_attention, paged_attention_forward, qk_norm_rope_store

pytestmark = pytest.mark.gpu
DEV = "cuda"
MAX_MISMATCH = 1e-4


def _rotated(w):
    qr, kr = onr.qk_norm_rope(w.q[None], w.k[None], w.q_weight, w.k_weight, w.cos[None], w.sin[None], w.eps)
    return qr[0].transpose(0, 1).contiguous(), kr[0].transpose(0, 1).contiguous()


def _check_rotated(got, ref, what):
    assert_close(got, ref, what=what)
    same = (got.cpu() == ref).float().mean().item()
    assert 1 - same <= MAX_MISMATCH, f"{what}: {1 - same:.2e} of elements differ"


def _store_all(kc, vc, pre, dec, kp, kd):
    """The oracle store of both halves into (kc, vc): the prefill tokens at
    positions 0..L-1, then each decode token at ctx-1."""
    cu = pre.cu_seqlens.tolist()
    for s, lst in enumerate(pre.block_lists):
        sl = slice(cu[s], cu[s + 1])
        ok.store_kv_cache(0, torch.tensor(lst), kp[sl].transpose(0, 1), pre.v[sl].transpose(0, 1), kc, vc)
    for i, lst in enumerate(dec.block_lists):
        ok.store_kv_cache(int(dec.positions[i]), torch.tensor(lst), kd[i][:, None], dec.v[i][:, None], kc, vc)


_REFS = {}


def _workload():
    if "w" not in _REFS:
        _REFS["w"] = W.make("qwen3-4b-mixed", poison=True)
    return _REFS["w"]


def _oracle_outputs(cpu):
    """The oracle's prefill and decode attention on its own rotated q/k and
    the oracle store of both halves (computed once per module)."""
    if "out" not in _REFS:
        pre, dec = cpu.prefill, cpu.decode
        qp_ref, kp_ref = _rotated(pre)
        qd_ref, kd_ref = _rotated(dec)
        kc_ref, vc_ref = cpu.k_cache.clone(), cpu.v_cache.clone()
        _store_all(kc_ref, vc_ref, pre, dec, kp_ref, kd_ref)
        ref_p = ov.flash_attn_varlen_func(qp_ref, kp_ref, pre.v, pre.cu_seqlens, pre.cu_seqlens, pre.max_seqlen,
                                          pre.max_seqlen, True)
        ref_d = op.paged_attention_forward(qd_ref, kc_ref, vc_ref, dec.block_tables, W.PAGE,
                                           dec.ctx_lens.to(torch.int32))
        _REFS["out"] = (ref_p, ref_d)
    return _REFS["out"]


def test_qwen3_4b_mixed_step_shared_pool():
    cpu = _workload()
    pre, dec = cpu.prefill, cpu.decode
    print(f"mixed step: {len(pre.seq_lens)} prefill seqs ({pre.q.shape[0]} tokens), {len(dec.ctx_lens)} decode seqs "
          f"(ctx {int(dec.ctx_lens.min())}..{int(dec.ctx_lens.max())}), pool {cpu.k_cache.shape[0]} pages",
          flush=True)
    g = cpu.to(DEV)
    gp, gd = g.prefill, g.decode
    kc, vc = g.k_cache, g.v_cache
    B = len(dec.ctx_lens)
    # ---- the step, in scheduler order, on one stream
    qp, kp = qk_norm_rope_store(gp.q, gp.k, gp.v, gp.q_weight, gp.k_weight, gp.cos, gp.sin, gp.eps, kc, vc,
                                gp.block_tables, gp.cu_seqlens)
    out_p = flash_attn_varlen_func(qp, kp, gp.v, gp.cu_seqlens, gp.cu_seqlens, gp.max_seqlen, gp.max_seqlen, True)
    qd, kd = qk_norm_rope_store(gd.q, gd.k, gd.v, gd.q_weight, gd.k_weight, gd.cos, gd.sin, gd.eps, kc, vc,
                                gd.block_tables, torch.arange(B + 1, dtype=torch.int32, device=DEV), gd.positions)
    out_d = paged_attention_forward(qd, kc, vc, gd.block_tables, W.PAGE, gd.ctx_lens.to(torch.int32))
    torch.cuda.synchronize()
    qp, kp, out_p, qd, kd, out_d = (t.cpu() for t in (qp, kp, out_p, qd, kd, out_d))
    kc_gpu, vc_gpu = kc.cpu(), vc.cpu()
    del g, gp, gd, kc, vc
    torch.cuda.empty_cache()

    # ---- rotated q/k of both halves
    qp_ref, kp_ref = _rotated(pre)
    qd_ref, kd_ref = _rotated(dec)
    _check_rotated(qp, qp_ref, "prefill q")
    _check_rotated(kp, kp_ref, "prefill k")
    _check_rotated(qd, qd_ref, "decode q")
    _check_rotated(kd, kd_ref, "decode k")

    # ---- both caches after both halves: exact, given the kernel's rotated K
    kc_exp, vc_exp = cpu.k_cache.clone(), cpu.v_cache.clone()
    _store_all(kc_exp, vc_exp, pre, dec, kp, kd)
    assert_bitexact(kc_gpu, kc_exp, "k_cache after prefill+decode")
    assert_bitexact(vc_gpu, vc_exp, "v_cache after prefill+decode")
    del kc_exp, vc_exp, kc_gpu, vc_gpu

    # ---- attention outputs, every sequence and head, on the oracle's own q/k
    ref_p, ref_d = _oracle_outputs(cpu)
    assert_close(out_p, ref_p, what="prefill attention, all 8 sequences")
    assert_close(out_d, ref_d, what=f"decode attention, all {B} sequences")


def _packed(gp, gd):
    """The tokens of both batches as one norm/RoPE/store call: prefill
    tokens first (positions 0..L-1 per sequence), then one token per decode
    sequence (position ctx-1); block tables padded to one width."""
    dev = gp.q.device
    T, B = gp.q.shape[0], gd.q.shape[0]
    width = max(gp.block_tables.shape[1], gd.block_tables.shape[1])

    def pad(t):
        return torch.nn.functional.pad(t, (0, width - t.shape[1]))

    ppos = torch.cat([torch.arange(int(n)) for n in gp.seq_lens.cpu()]).to(dev)
    return dict(
        q=torch.cat([gp.q, gd.q]), k=torch.cat([gp.k, gd.k]), v=torch.cat([gp.v, gd.v]),
        cos=torch.cat([gp.cos, gd.cos]), sin=torch.cat([gp.sin, gd.sin]),
        block_tables=torch.cat([pad(gp.block_tables), pad(gd.block_tables)]),
        cu_seqlens=torch.cat([gp.cu_seqlens, T + torch.arange(1, B + 1, dtype=torch.int32, device=dev)]),
        positions=torch.cat([ppos, gd.positions.to(dev)]).to(torch.int64),
    )


def _two_vs_one(cpu, **kw):
    """The step in scheduler order (two stores, two attention launches) and
    as one store + one attention launch; every output, the rotated q/k and
    both caches must match bit for bit -- except the prefill output of a
    group of 4 q-heads per kv head at head_dim 128, which the scheduler-order
    step computes with varlen_prefill_w64 and the one launch with
    varlen_prefill_gqa's body: the same arithmetic summed in another order,
    within one bf16 ulp. Returns the one-launch outputs."""
    gp0 = cpu.prefill
    w64 = (gp0.q.shape[1] // gp0.k.shape[1]) % 4 == 0 and gp0.q.shape[2] == 128
    runs = {}
    for mode in ("two", "one"):
        g = cpu.to(DEV)
        gp, gd = g.prefill, g.decode
        kc, vc = g.k_cache, g.v_cache
        T, B = gp.q.shape[0], gd.q.shape[0]
        sl = gd.ctx_lens.to(torch.int32)
        if mode == "two":
            qp, kp = qk_norm_rope_store(gp.q, gp.k, gp.v, gp.q_weight, gp.k_weight, gp.cos, gp.sin, gp.eps, kc, vc,
                                        gp.block_tables, gp.cu_seqlens)
            out_p = flash_attn_varlen_func(qp, kp, gp.v, gp.cu_seqlens, gp.cu_seqlens, gp.max_seqlen, gp.max_seqlen,
                                           True)
            qd, kd = qk_norm_rope_store(gd.q, gd.k, gd.v, gd.q_weight, gd.k_weight, gd.cos, gd.sin, gd.eps, kc, vc,
                                        gd.block_tables, torch.arange(B + 1, dtype=torch.int32, device=DEV),
                                        gd.positions)
            out_d = paged_attention_forward(qd, kc, vc, gd.block_tables, W.PAGE, sl)
            qr, kr = torch.cat([qp, qd]), torch.cat([kp, kd])
        else:
            pk = _packed(gp, gd)
            qr, kr = qk_norm_rope_store(pk["q"], pk["k"], pk["v"], gp.q_weight, gp.k_weight, pk["cos"], pk["sin"],
                                        gp.eps, kc, vc, pk["block_tables"], pk["cu_seqlens"], pk["positions"])
            out_p, out_d = mixed_attention(qr[:T], kr[:T], gp.v, gp.cu_seqlens, gp.max_seqlen, qr[T:], kc, vc,
                                           gd.block_tables, sl, **kw)
        torch.cuda.synchronize()
        runs[mode] = [t.cpu() for t in (out_p, out_d, qr, kr, kc, vc)]
        del g, gp, gd, kc, vc, qr, kr, out_p, out_d
        torch.cuda.empty_cache()
    names = ("prefill output", "decode output", "rotated q", "rotated k", "k_cache", "v_cache")
    for name, a, b in zip(names, runs["two"], runs["one"]):
        what = f"one store + one attention launch vs scheduler order: {name}"
        if name == "prefill output" and w64:
            assert_within_ulps(b, a, 1, what)
        else:
            assert_bitexact(b, a, what)
    return runs["one"]


def test_qwen3_4b_mixed_step_one_launch():
    cpu = _workload()
    print(f"mixed step, one attention launch: {len(cpu.prefill.seq_lens)} prefill + {len(cpu.decode.ctx_lens)} "
          f"decode seqs", flush=True)
    out_p, out_d = _two_vs_one(cpu, prefill_workgroups=256)[:2]  # one kernel (automatic would take two launches)
    ref_p, ref_d = _oracle_outputs(cpu)
    assert_close(out_p, ref_p, what="one launch: prefill attention, all 8 sequences")
    assert_close(out_d, ref_d, what=f"one launch: decode attention, all {len(cpu.decode.ctx_lens)} sequences")


def test_one_prefill_workgroup_many_items():
    """A single prefill workgroup takes every prefill item (6 sequences of
    200..600 tokens, 2 kv heads: over a hundred items, more than the 64 it
    resolves at a time), bit for bit against the scheduler-order step."""
    cpu = W.make_mixed("mixed-plan", 22, decode_batch=3, ctx_lo=1, ctx_hi=200, prefill_seqs=6, len_lo=200, len_hi=600,
                       num_heads=8, num_kv_heads=2, poison=True)
    items = sum((int(n) + 31) // 32 for n in cpu.prefill.seq_lens) * 2
    print(f"one prefill workgroup, {items} items", flush=True)
    assert items > 2 * 64
    _two_vs_one(cpu, prefill_workgroups=1)


@pytest.mark.parametrize("num_heads,num_kv_heads,prefill_workgroups",
                         [(8, 2, 0), (8, 2, 3), (8, 2, 1000), (8, 4, 0)])
def test_small_mixed_step_one_launch(num_heads, num_kv_heads, prefill_workgroups):
    """5 decode sequences (ctx 1..300) and 3 prefill sequences (1..150
    tokens, a short chunk) on one pool: 4 q-heads per kv head take the one
    kernel (automatically with one prefill workgroup per CU, and asked for
    with 3 and 1000, more than fit beside the decode ones); 2 take the
    two-launch fallback."""
    cpu = W.make_mixed("mixed-small", 21, decode_batch=5, ctx_lo=1, ctx_hi=300, prefill_seqs=3, len_lo=1, len_hi=150,
                       num_heads=num_heads, num_kv_heads=num_kv_heads, poison=True)
    print(f"small mixed step: heads {num_heads}/{num_kv_heads}, prefill_workgroups {prefill_workgroups}", flush=True)
    _two_vs_one(cpu, prefill_workgroups=prefill_workgroups)
