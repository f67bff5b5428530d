"""Pins for the oracle's paged decode and varlen prefill attention (CPU).

Paged decode (oracle.paged, restating paged_attention.py:8-121):
* float64 brute force -- gather each sequence's tokens, softmax, weighted sum
  -- on the reference test's three configurations and others, fp32 inputs,
  1e-5 (the same math as tests/model/test_paged_attention_kernel.py:26-64);
* seq_len 1 returns the V row exactly; all-equal K gives the uniform mean of V;
* GQA group 1 equals per-head SDPA; a page as long as the context equals
  contiguous SDPA;
* poisoned (1e4) and NaN slots past seq_len do not leak
  (test_paged_attention_kernel.py:187-222);
* the reference's CPU decode branch (qwen3.py:359-385) -- per-token gather
  loop, repeat_interleave, SDPA -- agrees;
* the "3D" guard.

Varlen prefill (oracle.varlen, restating varlen_attention.py:8-142):
* float64 brute force with the kernel's top-left causal mask, also when
  q_len != k_len; the reference's own naive check (:224-254) for equal
  lengths; the block-diagonal-mask SDPA CPU branch (qwen3.py:132-171);
* length-1 sequences return V; row 0 of a causal sequence returns v[0];
* the reference self-test configuration (fp16, seed 42, :257-307) at its own
  tolerances; the guards.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import paged as op
from oracle import varlen as ov


def _paged_inputs(lens, hq, hkv, d, bs, dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    bps = [max(1, math.ceil(n / bs)) for n in lens]
    nb = sum(bps) + 3
    q = torch.randn(len(lens), hq, d, generator=g).to(dtype)
    kc = torch.randn(nb, hkv, bs, d, generator=g).to(dtype)
    vc = torch.randn(nb, hkv, bs, d, generator=g).to(dtype)
    perm = torch.randperm(nb, generator=g)
    bt = torch.zeros(len(lens), max(bps), dtype=torch.int32)
    cur = 0
    for s, n in enumerate(bps):
        bt[s, :n] = perm[cur : cur + n]
        cur += n
    return q, kc, vc, bt, torch.tensor(lens, dtype=torch.int32)


def paged_brute(q, kc, vc, bt, bs, sl):
    S, H, D = q.shape
    G = H // kc.shape[1]
    out = torch.empty(S, H, D, dtype=torch.float64)
    for s in range(S):
        L = int(sl[s])
        blocks = [int(bt[s, t // bs]) for t in range(L)]
        slots = [t % bs for t in range(L)]
        K, V = kc[blocks, :, slots, :].double(), vc[blocks, :, slots, :].double()
        for h in range(H):
            p = torch.softmax((K[:, h // G] @ q[s, h].double()) / math.sqrt(D), 0)
            out[s, h] = p @ V[:, h // G]
    return out


PAGED_CASES = [
    (4, 4, 64, 16, [10]),
    (8, 2, 64, 16, [7, 16, 40]),
    (16, 4, 128, 32, [1, 33, 64]),
    (32, 8, 128, 16, [1000, 17, 513]),
    (8, 8, 128, 4, [9, 2, 30]),
]


@pytest.mark.parametrize("case", range(len(PAGED_CASES)))
def test_paged_vs_fp64(case):
    hq, hkv, d, bs, lens = PAGED_CASES[case]
    q, kc, vc, bt, sl = _paged_inputs(lens, hq, hkv, d, bs, seed=case)
    out = op.paged_attention_forward(q, kc, vc, bt, bs, sl)
    assert (out.double() - paged_brute(q, kc, vc, bt, bs, sl)).abs().max() < 1e-5


def test_paged_special_cases():
    q, kc, vc, bt, sl = _paged_inputs([1, 1], 8, 2, 64, 16, seed=1)
    out = op.paged_attention_forward(q, kc, vc, bt, 16, sl)
    for s in range(2):
        for h in range(8):
            assert torch.allclose(out[s, h], vc[int(bt[s, 0]), h // 4, 0], atol=0, rtol=0)
    # all-equal keys: uniform weights -> mean of the V rows
    q, kc, vc, bt, sl = _paged_inputs([37], 4, 1, 64, 16, seed=2)
    kc[:] = kc[0, 0, 0]
    out = op.paged_attention_forward(q, kc, vc, bt, 16, sl)
    blocks = [int(bt[0, t // 16]) for t in range(37)]
    mean_v = vc[blocks, 0, [t % 16 for t in range(37)]].mean(0)
    assert (out[0] - mean_v).abs().max() < 1e-5


def test_paged_mha_and_single_page_equal_sdpa():
    q, kc, vc, bt, sl = _paged_inputs([50], 4, 4, 64, 64, seed=3)  # one page holds the context
    out = op.paged_attention_forward(q, kc, vc, bt, 64, sl)
    page = int(bt[0, 0])
    k = kc[page, :, :50][None]
    v = vc[page, :, :50][None]
    ref = F.scaled_dot_product_attention(q[0][None, :, None], k, v)[0, :, 0]
    assert (out[0] - ref).abs().max() < 1e-5


def test_paged_poison_does_not_leak():
    q, kc, vc, bt, sl = _paged_inputs([5, 21], 8, 2, 64, 16, seed=4)
    ref = op.paged_attention_forward(q, kc, vc, bt, 16, sl)
    kc[int(bt[0, 0]), :, 5:] = 1e4
    vc[int(bt[0, 0]), :, 5:] = 1e4
    kc[int(bt[1, 1]), :, 5:] = float("nan")
    vc[int(bt[1, 1]), :, 5:] = float("inf")
    assert torch.equal(op.paged_attention_forward(q, kc, vc, bt, 16, sl), ref)


@pytest.mark.parametrize("literal", [True, False])
def test_reference_cpu_decode_path_agrees(literal):
    q, kc, vc, bt, sl = _paged_inputs([33, 7, 100], 16, 4, 128, 16, seed=5)
    out = op.paged_attention_forward(q, kc, vc, bt, 16, sl)
    tables = [bt[s, : math.ceil(int(sl[s]) / 16)].tolist() for s in range(3)]
    cpu = op.decode_cpu_path(q.transpose(0, 1)[None], kc, vc, tables, [int(n) - 1 for n in sl], literal_gather=literal)
    assert (cpu - out).abs().max() < 1e-5


def test_paged_guard():
    with pytest.raises(ValueError, match="3D"):
        op.paged_attention_forward(torch.zeros(4, 64), torch.zeros(2, 4, 16, 64), torch.zeros(2, 4, 16, 64),
                                   torch.zeros(1, 1, dtype=torch.int32), 16, torch.ones(1, dtype=torch.int32))


# ------------------------------------------------------------------ varlen --
def varlen_brute(q, k, v, cq, ck, causal, scale):
    """float64, top-left causal (key j visible to query i iff j <= i)."""
    out = torch.zeros(q.shape, dtype=torch.float64)
    G = q.shape[1] // k.shape[1]
    for b in range(len(cq) - 1):
        qs, qe, ks, ke = int(cq[b]), int(cq[b + 1]), int(ck[b]), int(ck[b + 1])
        for h in range(q.shape[1]):
            s = (q[qs:qe, h].double() @ k[ks:ke, h // G].double().T) * scale
            if causal:
                i = torch.arange(qe - qs)[:, None]
                j = torch.arange(ke - ks)[None, :]
                s = s.masked_fill(j > i, float("-inf"))
            out[qs:qe, h] = torch.softmax(s, -1) @ v[ks:ke, h // G].double()
    return out


def _cu(lens):
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    return cu


def _varlen_inputs(lq, lk, hq, hkv, d, dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(sum(lq), hq, d, generator=g).to(dtype), torch.randn(sum(lk), hkv, d, generator=g).to(dtype),
            torch.randn(sum(lk), hkv, d, generator=g).to(dtype), _cu(lq), _cu(lk))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("lens", [([5, 33, 70, 1], None), ([5, 40, 64], [9, 33, 100])])
def test_varlen_vs_fp64(causal, lens):
    lq, lk = lens[0], lens[1] or lens[0]
    q, k, v, cq, ck = _varlen_inputs(lq, lk, 8, 2, 64, seed=1)
    out = ov.flash_attn_varlen_func(q, k, v, cq, ck, max(lq), max(lk), causal)
    assert (out.double() - varlen_brute(q, k, v, cq, ck, causal, 64**-0.5)).abs().max() < 1e-5
    if lens[1] is None:
        naive = ov.reference_attn_varlen(q.double(), k.double(), v.double(), cq, ck, causal, 64**-0.5)
        assert (out.double() - naive).abs().max() < 1e-5


def test_varlen_block_mask_sdpa_agrees():
    lens = [17, 3, 64]
    q, k, v, cu, _ = _varlen_inputs(lens, lens, 8, 4, 128, seed=2)
    out = ov.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), True)
    sdpa = ov.prefill_sdpa_block_mask(q.transpose(0, 1)[None], k.transpose(0, 1)[None], v.transpose(0, 1)[None],
                                      lens, 128)
    assert (out.reshape(1, sum(lens), -1) - sdpa).abs().max() < 1e-5
    per_seq = ov.prefill_sdpa_per_sequence(q, k, v, cu)  # the vectorised CPU baseline
    assert (out - per_seq).abs().max() < 1e-5
    assert torch.equal(per_seq.reshape(1, sum(lens), -1), sdpa) or (per_seq.reshape(1, sum(lens), -1) - sdpa).abs().max() < 1e-6


def test_varlen_special_cases():
    q, k, v, cu, _ = _varlen_inputs([1, 1, 1], [1, 1, 1], 4, 2, 64, seed=3)
    out = ov.flash_attn_varlen_func(q, k, v, cu, cu, 1, 1, True)
    assert torch.equal(out, v[:, [0, 0, 1, 1]])
    q, k, v, cu, _ = _varlen_inputs([40], [40], 4, 4, 64, seed=4)
    out = ov.flash_attn_varlen_func(q, k, v, cu, cu, 40, 40, True)
    assert (out[0] - v[0]).abs().max() < 1e-6


@pytest.mark.parametrize("causal", [True, False])
def test_varlen_reference_selftest_config(causal):
    """fp16, seed 42, 4 sequences U[32,256], 16/4 heads, D 64 (varlen_attention.py:257-307)."""
    torch.manual_seed(42)
    lens = torch.randint(32, 257, (4,)).tolist()
    q, k, v, cu, _ = _varlen_inputs(lens, lens, 16, 4, 64, dtype=torch.float16, seed=42)
    out = ov.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), causal, 1 / 8)
    ref = ov.reference_attn_varlen(q, k, v, cu, cu, causal, 1 / 8)
    d = (out.float() - ref.float()).abs()
    assert d.max() < 5e-2 and d.mean() < 1e-3


def test_varlen_guards():
    with pytest.raises(ValueError, match="3D"):
        ov.flash_attn_varlen_func(torch.zeros(4, 64), torch.zeros(4, 1, 64), torch.zeros(4, 1, 64), _cu([4]), _cu([4]),
                                  4, 4, True)
    with pytest.raises(ValueError, match="divisible"):
        ov.flash_attn_varlen_func(torch.zeros(4, 3, 64), torch.zeros(4, 2, 64), torch.zeros(4, 2, 64), _cu([4]),
                                  _cu([4]), 4, 4, True)
