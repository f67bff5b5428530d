"""The oracle's pins catch plausible mistakes (CPU).

Each case plants one mistake in a copy of an oracle function -- a dropped term,
a wrong sign or index, a transposed mask, a moved rounding point -- by editing
its source text, and checks that the comparison that pins the real function
(transformers on the CPU, float64 brute force, the reference's store cases)
rejects the mutant. The real functions are untouched.
"""

import inspect
import math
import textwrap

import pytest
import torch
from transformers import Qwen3Config
from transformers.models.qwen3 import modeling_qwen3 as hf

from oracle import kv_store as ok
from oracle import norm_rope as onr
from oracle import paged as op
from oracle import varlen as ov
from tests.test_oracle_attention import _cu, _paged_inputs, _varlen_inputs, paged_brute, varlen_brute

D = 128


def mutate(func, old: str, new: str, *more: str):
    """A copy of ``func`` with ``old`` replaced by ``new`` (and further
    old/new pairs in ``more``) in its source."""
    src = textwrap.dedent(inspect.getsource(func))
    pairs = [(old, new)] + list(zip(more[0::2], more[1::2]))
    for o, n in pairs:
        assert o in src, f"mutation anchor {o!r} not found in {func.__name__}"
        src = src.replace(o, n, 1)
    ns = dict(func.__globals__)
    exec(compile(src, f"<mutant {func.__name__}>", "exec"), ns)
    return ns[func.__name__]


# ----------------------------------------------------------- RMSNorm / RoPE --
def _norm_inputs(scale=1.0):
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(1, 9, 8, D, generator=g) * scale).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    mod = hf.Qwen3RMSNorm(D, eps=1e-6).to(torch.bfloat16)
    mod.weight.data.copy_(w)
    return x, w, mod


@pytest.mark.parametrize("old,new,scale", [
    ("variance + eps", "variance", 1e-3),                                  # dropped eps
    ("return weight * h.to(input_dtype)", "return (weight * h).to(input_dtype)", 1.0),  # rounding point moved
    ("mean(-1, keepdim=True)", "sum(-1, keepdim=True) / (h.shape[-1] - 1)", 1.0),   # wrong mean
])
def test_rms_norm_mutants_caught(old, new, scale):
    x, w, mod = _norm_inputs(scale)
    assert torch.equal(onr.rms_norm(x, w, 1e-6), mod(x))
    bad = mutate(onr.rms_norm, old, new)
    assert not torch.equal(bad(x, w, 1e-6), mod(x))


def _rope_ref():
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 4, 7, D, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 2, 7, D, generator=g).to(torch.bfloat16)
    cfg = Qwen3Config(head_dim=D, hidden_size=D * 8, num_attention_heads=8, num_key_value_heads=8, rope_theta=1e6,
                      max_position_embeddings=1 << 20)
    c, s = hf.Qwen3RotaryEmbedding(cfg)(torch.empty(0, dtype=torch.bfloat16), torch.arange(50, 57)[None])
    return q, k, c, s, hf.apply_rotary_pos_emb(q, k, c, s)


@pytest.mark.parametrize("old,new", [
    ("torch.cat((-x2, x1), dim=-1)", "torch.cat((x2, -x1), dim=-1)"),      # sign of rotate_half
    ("torch.cat((-x2, x1), dim=-1)", "torch.stack((-x[..., 1::2], x[..., 0::2]), -1).flatten(-2)"),  # interleaved
])
def test_rotate_half_mutants_caught(old, new, monkeypatch):
    q, k, c, s, (qr, kr) = _rope_ref()
    monkeypatch.setattr(onr, "rotate_half", mutate(onr.rotate_half, old, new))
    q2, _ = onr.apply_rotary_pos_emb(q, k, c, s)
    assert not torch.equal(q2, qr)


@pytest.mark.parametrize("old,new", [
    ("q_embed = (q * cos) + (rotate_half(q) * sin)", "q_embed = (q * sin) + (rotate_half(q) * cos)"),  # cos/sin swapped
    ("q_embed = (q * cos) + (rotate_half(q) * sin)", "q_embed = (q * cos) - (rotate_half(q) * sin)"),  # sign
])
def test_apply_rotary_mutants_caught(old, new):
    q, k, c, s, (qr, kr) = _rope_ref()
    q2, _ = mutate(onr.apply_rotary_pos_emb, old, new)(q, k, c, s)
    assert not torch.equal(q2, qr)


def test_rope_frequency_mutant_caught():
    cfg = Qwen3Config(head_dim=D, hidden_size=D * 8, num_attention_heads=8, num_key_value_heads=8, rope_theta=1e6,
                      max_position_embeddings=1 << 20)
    pos = torch.arange(0, 4000, 97)[None]
    c_ref, _ = hf.Qwen3RotaryEmbedding(cfg)(torch.empty(0, dtype=torch.float32), pos)
    bad = mutate(onr.rope_inv_freq, "/ head_dim))", "/ (head_dim - 2)))")
    c_bad = torch.cat([torch.outer(pos[0].float(), bad(D, 1e6))] * 2, -1).cos()
    assert not torch.equal(c_bad, c_ref[0])


# ------------------------------------------------------------------ store --
@pytest.mark.parametrize("old,new", [
    ("slot = pos % block_size", "slot = (pos + 1) % block_size"),      # off-by-one slot
    ("blk = bt[pos // block_size]", "blk = bt[pos % len(bt)]"),         # wrong block index
])
def test_store_mutants_caught(old, new):
    from tests.test_oracle_store import REF_CASES, _brute

    hkv, bs, d, nb, seqs = REF_CASES[4]
    g = torch.Generator().manual_seed(4)
    ks = [torch.randn(hkv, s["seq_len"], d, generator=g) for s in seqs]
    shape = (nb, hkv, bs, d)
    bad = mutate(ok.store_kv_cache, old, new)
    kp, vp = torch.zeros(shape), torch.zeros(shape)
    for s, k in zip(seqs, ks):
        bad(s["start_pos"], torch.tensor(s["block_table"]), k, k, kp, vp)
    assert not torch.equal(kp, _brute(seqs, ks, shape))


# ------------------------------------------------------------ paged decode --
@pytest.mark.parametrize("old,new", [
    ("kv_head = torch.arange(num_heads) // group", "kv_head = torch.arange(num_heads) % num_kv_heads"),  # GQA map
    ("scale = 1.0 / math.sqrt(head_dim)", "scale = 1.0"),                                            # no scale
    ("qk = torch.where(valid[:, None, :], qk, float(\"-inf\"))  # :103-105", "pass"),                 # no mask
    ("alpha = torch.exp(m - m_new)  # :109", "alpha = torch.exp(m_new - m)"),                       # rescale sign
])
def test_paged_mutants_caught(old, new):
    q, kc, vc, bt, sl = _paged_inputs([7, 16, 40], 8, 2, 64, 16, seed=0)
    ref = paged_brute(q, kc, vc, bt, 16, sl)
    assert (op.paged_attention_forward(q, kc, vc, bt, 16, sl).double() - ref).abs().max() < 1e-5
    out = mutate(op.paged_attention_forward, old, new)(q, kc, vc, bt, 16, sl).double()
    assert not ((out - ref).abs().max() < 1e-5)


def test_paged_dropped_load_mask_caught():
    """Dropping the masked K load alone is covered by the score mask; dropping the
    masked loads and the score mask together must show (slots past seq_len)."""
    q, kc, vc, bt, sl = _paged_inputs([7, 16, 40], 8, 2, 64, 16, seed=0)
    ref = paged_brute(q, kc, vc, bt, 16, sl)
    bad = mutate(op.paged_attention_forward,
                 "k = torch.where(valid[:, None, :, None], k, 0.0)  # masked load, other=0", "pass",
                 "v = torch.where(valid[:, None, :, None], v, 0.0)", "pass",
                 'qk = torch.where(valid[:, None, :], qk, float("-inf"))  # :103-105', "pass")
    assert not ((bad(q, kc, vc, bt, 16, sl).double() - ref).abs().max() < 1e-5)


# ---------------------------------------------------------- varlen prefill --
@pytest.mark.parametrize("old,new", [
    ("mask = mask & (rows[:, None] >= cols[None, :])", "mask = mask & (rows[:, None] <= cols[None, :])"),  # transposed
    ("kv_head = torch.arange(num_heads_q) // group", "kv_head = torch.arange(num_heads_q) % num_heads_k"),
    ("softmax_scale = 1.0 / (head_dim**0.5)", "softmax_scale = 1.0"),
    ("l = l * alpha + p.sum(-1)", "l = l + p.sum(-1)"),                                                    # no rescale
])
def test_varlen_mutants_caught(old, new):
    lens = [5, 33, 70, 1]
    q, k, v, cu, _ = _varlen_inputs(lens, lens, 8, 2, 64, seed=1)
    ref = varlen_brute(q, k, v, cu, cu, True, 64**-0.5)
    assert (ov.flash_attn_varlen_func(q, k, v, cu, cu, 70, 70, True).double() - ref).abs().max() < 1e-5
    bad = mutate(ov.flash_attn_varlen_func, old, new)
    out = bad(q, k, v, cu, cu, 70, 70, True).double()
    assert not ((out - ref).abs().max() < 1e-5)
