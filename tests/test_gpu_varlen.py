"""Varlen causal prefill on the GPU vs the oracle.

The oracle restates the reference kernel (varlen_attention.py:8-142): 32-key
online softmax, top-left causal mask, P rounded to the V dtype before P.V.
Cases: the reference's self-test configuration (varlen_attention.py:257-307:
fp16, seed 42, 4 sequences of U[32,256] tokens, 16/4 heads, D 64, causal and
not), bf16/fp16/fp32, GQA groups, q_len != k_len, length-1 sequences, the
call site's strided (T, H, D) views (qwen3.py:199-201), and the full
Qwen3-8B-shaped 16-sequence prefill, every sequence and head.
Tolerance: max-abs 2e-2, mean-abs 2e-3 for 16-bit dtypes (the reference's
own fp16 check is max 5e-2, mean 1e-3); fp32 1e-4.
"""

import math

import pytest
import torch

from oracle import varlen as ov
from tests.helpers import assert_close
from tinyserver_amd import workloads as W
from tinyserver_amd.kernels import flash_attn_varlen_func

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cu(lens):
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    return cu


def _inputs(lens_q, lens_k, hq, hkv, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(sum(lens_q), hq, d, generator=g).to(dtype)
    k = torch.randn(sum(lens_k), hkv, d, generator=g).to(dtype)
    v = torch.randn(sum(lens_k), hkv, d, generator=g).to(dtype)
    return q, k, v, _cu(lens_q), _cu(lens_k)


def _tol(dtype):
    return dict(max_abs=1e-4, mean_abs=1e-5) if dtype == torch.float32 else {}


@pytest.mark.parametrize("causal", [True, False])
def test_reference_selftest_config(causal):
    torch.manual_seed(42)
    lens = torch.randint(32, 257, (4,)).tolist()
    q, k, v, cu, _ = _inputs(lens, lens, 16, 4, 64, torch.float16, seed=42)
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), cu.to(DEV), max(lens), max(lens),
                                 causal=causal, softmax_scale=1.0 / math.sqrt(64))
    torch.cuda.synchronize()
    ref = ov.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), causal, 1.0 / math.sqrt(64))
    assert_close(out, ref, what=f"selftest causal={causal}")
    # and the reference's own looser check against its naive restatement
    naive = ov.reference_attn_varlen(q.float(), k.float(), v.float(), cu, cu, causal, 1.0 / math.sqrt(64))
    assert_close(out, naive, max_abs=5e-2, mean_abs=1e-3, what="vs naive")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("group", [1, 4, 8])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_matches_oracle(dtype, group, head_dim):
    lens = [1, 31, 32, 33, 100, 257]
    q, k, v, cu, _ = _inputs(lens, lens, 2 * group, 2, head_dim, dtype, seed=group)
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), cu.to(DEV), max(lens), max(lens), True)
    torch.cuda.synchronize()
    ref = ov.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), True)
    assert_close(out, ref, what=f"{dtype} G={group} D={head_dim}", **_tol(dtype))


@pytest.mark.parametrize("group,head_dim", [(2, 64), (3, 128), (16, 128), (32, 64)])
def test_other_group_sizes(group, head_dim):
    """Groups that divide 16 take the LDS-staged kernel; others the per-head kernel."""
    lens = [17, 64, 200, 5]
    q, k, v, cu, _ = _inputs(lens, lens, 2 * group, 2, head_dim, torch.bfloat16, seed=10 + group)
    for causal in (True, False):
        out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), cu.to(DEV), max(lens), max(lens),
                                     causal)
        torch.cuda.synchronize()
        ref = ov.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), causal)
        assert_close(out, ref, what=f"G={group} D={head_dim} causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
def test_q_len_differs_from_k_len(causal):
    lq, lk = [5, 40, 64], [9, 33, 100]
    q, k, v, cq, ck = _inputs(lq, lk, 8, 2, 128, torch.bfloat16, seed=3)
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cq.to(DEV), ck.to(DEV), max(lq), max(lk), causal)
    torch.cuda.synchronize()
    ref = ov.flash_attn_varlen_func(q, k, v, cq, ck, max(lq), max(lk), causal)
    assert_close(out, ref, what=f"lq!=lk causal={causal}")


def test_sequence_without_keys():
    """A sequence with queries but no keys: 0/0 (NaN) rows, as the reference's
    l = 0 division gives; the other sequence is unaffected."""
    lq, lk = [16, 40], [0, 50]
    q, k, v, cq, ck = _inputs(lq, lk, 8, 2, 128, torch.bfloat16, seed=13)
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cq.to(DEV), ck.to(DEV), max(lq), max(lk),
                                 False).cpu()
    ref = ov.flash_attn_varlen_func(q, k, v, cq, ck, max(lq), max(lk), False)
    assert torch.isnan(ref[:16]).all() and torch.isnan(out[:16]).all()
    assert_close(out[16:], ref[16:], what="sequence after an empty one")


def test_repeated_calls_are_identical():
    """Many calls in a row, two shapes interleaved: the persistent
    workgroups compute every work item exactly once, in a fixed assignment, so
    every output is bit-identical to the first call's."""
    lens_a, lens_b = [300, 17, 1000, 64], [33, 700]
    qa, ka, va, ca, _ = _inputs(lens_a, lens_a, 32, 8, 128, torch.bfloat16, seed=21)
    qb, kb, vb, cb, _ = _inputs(lens_b, lens_b, 32, 8, 128, torch.bfloat16, seed=22)
    qa, ka, va, ca = qa.to(DEV), ka.to(DEV), va.to(DEV), ca.to(DEV)
    qb, kb, vb, cb = qb.to(DEV), kb.to(DEV), vb.to(DEV), cb.to(DEV)
    first_a = flash_attn_varlen_func(qa, ka, va, ca, ca, max(lens_a), max(lens_a), True)
    first_b = flash_attn_varlen_func(qb, kb, vb, cb, cb, max(lens_b), max(lens_b), True)
    for _ in range(40):
        oa = flash_attn_varlen_func(qa, ka, va, ca, ca, max(lens_a), max(lens_a), True)
        ob = flash_attn_varlen_func(qb, kb, vb, cb, cb, max(lens_b), max(lens_b), True)
        assert torch.equal(oa, first_a) and torch.equal(ob, first_b)
    ref = ov.flash_attn_varlen_func(qa.cpu(), ka.cpu(), va.cpu(), ca.cpu(), ca.cpu(), max(lens_a), max(lens_a), True)
    assert_close(first_a.cpu(), ref, what="repeated calls")


def test_single_token_sequences_return_v():
    lens = [1, 1, 1]
    q, k, v, cu, _ = _inputs(lens, lens, 8, 2, 128, torch.bfloat16, seed=5)
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), cu.to(DEV), 1, 1, True).cpu()
    for t in range(3):
        for h in range(8):
            assert torch.equal(out[t, h], v[t, h // 4])


def test_call_site_strided_views():
    """q/k/v as (1, H, T, D) tensors squeezed and transposed, as qwen3.py:199-201 passes them."""
    lens = [70, 129, 3]
    q, k, v, cu, _ = _inputs(lens, lens, 16, 8, 128, torch.bfloat16, seed=6)
    qh = q.transpose(0, 1).contiguous()[None].to(DEV)  # (1, Hq, T, D)
    kh = k.transpose(0, 1).contiguous()[None].to(DEV)
    vh = v.transpose(0, 1).contiguous()[None].to(DEV)
    out = flash_attn_varlen_func(qh.squeeze(0).transpose(0, 1), kh.squeeze(0).transpose(0, 1),
                                 vh.squeeze(0).transpose(0, 1), cu.to(DEV), cu.to(DEV), max(lens), max(lens),
                                 causal=True, softmax_scale=128**-0.5)
    torch.cuda.synchronize()
    ref = ov.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), True, 128**-0.5)
    assert_close(out, ref, what="strided views")


def test_qwen3_8b_prefill_full():
    """The Qwen3-8B 16-sequence prefill, every sequence and every head."""
    w = W.make("qwen3-8b-prefill-16seq", device=DEV)
    out = flash_attn_varlen_func(w.q, w.k, w.v, w.cu_seqlens, w.cu_seqlens, w.max_seqlen, w.max_seqlen, True)
    torch.cuda.synchronize()
    print(f"{w.name}: {w.q.shape[0]} tokens, oracle on the CPU", flush=True)
    cu = w.cu_seqlens.cpu()
    ref = ov.flash_attn_varlen_func(w.q.cpu(), w.k.cpu(), w.v.cpu(), cu, cu, w.max_seqlen, w.max_seqlen, True)
    assert_close(out, ref, what="Qwen3-8B prefill, all 16 sequences x 32 heads")


def test_long_sequence_sampled_rows():
    """An 8192-token causal sequence (256 query tiles, up to 256 key blocks
    each) beside a short one, checked on sampled query rows against fp64
    softmax attention over the row's visible keys."""
    lens = [8192, 100]
    q, k, v, cq, _ = _inputs(lens, lens, 32, 8, 128, torch.bfloat16, seed=41)
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cq.to(DEV), cq.to(DEV), max(lens), max(lens),
                                 True).cpu().double()
    scale = 128 ** -0.5
    got, want = [], []
    for r, start in [(0, 0), (31, 0), (32, 0), (4095, 0), (8160, 0), (8191, 0), (8192, 8192), (8291, 8192)]:
        for h in (0, 17, 31):
            kk, vv = k[start:r + 1, h // 4].double(), v[start:r + 1, h // 4].double()
            p = torch.softmax((kk @ q[r, h].double()) * scale, 0)
            want.append(p @ vv)
            got.append(out[r, h])
    assert_close(torch.stack(got), torch.stack(want), what="long sequence, sampled rows")


def test_many_short_sequences():
    """1000 sequences of 1-64 tokens (a wide, shallow batch) against the oracle."""
    g = torch.Generator().manual_seed(43)
    lens = torch.randint(1, 65, (1000,), generator=g).tolist()
    q, k, v, cq, ck = _inputs(lens, lens, 32, 8, 128, torch.bfloat16, seed=44)
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cq.to(DEV), ck.to(DEV), max(lens), max(lens),
                                 True).cpu()
    ref = ov.flash_attn_varlen_func(q, k, v, cq, ck, max(lens), max(lens), True)
    assert_close(out, ref, what="1000 short sequences")


def _run(lens, q, k, v, causal=True):
    cu = _cu(lens).to(DEV)
    return flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cu, cu, max(lens), max(lens), causal).cpu()


def test_item_plan_limits_match():
    """The persistent kernel resolves work items from a per-workgroup plan
    for calls of at most 64 sequences and 256 query tiles per sequence, and
    by a wave-cooperative search otherwise. A call just past each limit (65
    sequences; a sequence of 257 tiles) must give its other sequences the
    same bits as a call within the limit, and the 64-sequence call must match
    the oracle."""
    g = torch.Generator().manual_seed(45)
    lens = torch.randint(1, 201, (65,), generator=g).tolist()
    q, k, v, _, _ = _inputs(lens, lens, 32, 8, 128, torch.bfloat16, seed=46)
    t64 = sum(lens[:64])
    print(f"65 vs 64 sequences ({sum(lens)} / {t64} tokens)", flush=True)
    out65 = _run(lens, q, k, v)
    out64 = _run(lens[:64], q[:t64], k[:t64], v[:t64])
    assert torch.equal(out65[:t64], out64), "65-sequence call vs 64-sequence call"
    ref = ov.flash_attn_varlen_func(q[:t64], k[:t64], v[:t64], _cu(lens[:64]), _cu(lens[:64]), max(lens[:64]),
                                    max(lens[:64]), True)
    assert_close(out64, ref, what="64 sequences vs oracle")

    lens = [40, 300, 8193]  # 257 query tiles in the last sequence
    q, k, v, _, _ = _inputs(lens, lens, 32, 8, 128, torch.bfloat16, seed=47)
    print("a 257-tile sequence beside two short ones", flush=True)
    out_long = _run(lens, q, k, v)
    out_short = _run(lens[:2], q[:340], k[:340], v[:340])
    assert torch.equal(out_long[:340], out_short), "short sequences beside a 257-tile one vs alone"
    scale = 128 ** -0.5
    got, want = [], []
    for r in (340, 340 + 8191, 340 + 8192):
        for h in (0, 31):
            kk, vv = k[340:r + 1, h // 4].double(), v[340:r + 1, h // 4].double()
            p = torch.softmax((kk @ q[r, h].double()) * scale, 0)
            want.append(p @ vv)
            got.append(out_long[r, h].double())
    assert_close(torch.stack(got), torch.stack(want), what="257-tile sequence, sampled rows")
