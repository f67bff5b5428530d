"""Pins for the oracle's QK RMSNorm and RoPE (CPU).

The arithmetic lives in transformers 5.15.0 (models/qwen3/modeling_qwen3.py),
which the reference imports; it is not under the reference tree. The oracle is
pinned (a) bit-exactly against those installed functions, called on the CPU
as the reference's call site calls them (server/model/patches/qwen3.py:264-287),
and (b) against closed forms computed in float64: the RMSNorm definition, RoPE
at position 0 being the identity, RoPE preserving each (i, i+D/2) pair's norm,
and RoPE(a) then RoPE(b) equal to RoPE(a+b).

Also pinned: the fp32 order of mean(x^2) in the CPU reduction, which the HIP
kernel reproduces -- four 8-wide accumulators over 32-element strides, added
in order, then the 8 lanes in order.
"""

import math

import numpy as np
import pytest
import torch
from transformers import Qwen3Config
from transformers.models.qwen3 import modeling_qwen3 as hf

from oracle import norm_rope as onr

D = 128


def _hf_rotary(theta=1e6, head_dim=D):
    cfg = Qwen3Config(head_dim=head_dim, hidden_size=head_dim * 8, num_attention_heads=8, num_key_value_heads=8,
                      rope_theta=theta, max_position_embeddings=1 << 20)
    return hf.Qwen3RotaryEmbedding(cfg)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rms_norm_matches_transformers(dtype):
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(1, 37, 16, D, generator=g) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    mod = hf.Qwen3RMSNorm(D, eps=1e-6).to(dtype)
    mod.weight.data.copy_(w)
    assert torch.equal(onr.rms_norm(x, w, 1e-6), mod(x))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_cos_sin_matches_transformers(dtype):
    pos = torch.tensor([[0, 1, 2, 15, 16, 511, 4095, 8191, 32767, 40959]])
    c_ref, s_ref = _hf_rotary()(torch.empty(0, dtype=dtype), pos)
    c, s = onr.rope_cos_sin(pos, D, 1e6, dtype)
    assert torch.equal(c, c_ref) and torch.equal(s, s_ref)


def test_apply_rotary_matches_transformers():
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 16, 9, D, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 8, 9, D, generator=g).to(torch.bfloat16)
    c, s = onr.rope_cos_sin(torch.arange(100, 109)[None], D, 1e6, torch.bfloat16)
    a1, b1 = hf.apply_rotary_pos_emb(q, k, c, s)
    a2, b2 = onr.apply_rotary_pos_emb(q, k, c, s)
    assert torch.equal(a1, a2) and torch.equal(b1, b2)


def test_call_site_sequence_matches_transformers():
    """q_norm/k_norm modules, transpose, apply_rotary_pos_emb -- qwen3.py:264-287."""
    g = torch.Generator().manual_seed(2)
    T, hq, hkv = 21, 16, 8
    q = torch.randn(1, T, hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(1, T, hkv, D, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    pos = torch.randint(0, 30000, (1, T), generator=g)
    cos, sin = _hf_rotary()(torch.empty(0, dtype=torch.bfloat16), pos)
    qn, kn = hf.Qwen3RMSNorm(D, 1e-6).to(torch.bfloat16), hf.Qwen3RMSNorm(D, 1e-6).to(torch.bfloat16)
    qn.weight.data.copy_(qw)
    kn.weight.data.copy_(kw)
    qr, kr = hf.apply_rotary_pos_emb(qn(q).transpose(1, 2), kn(k).transpose(1, 2), cos, sin)
    q2, k2 = onr.qk_norm_rope(q, k, qw, kw, cos, sin, 1e-6)
    assert torch.equal(q2, qr) and torch.equal(k2, kr)


def test_rms_norm_closed_form_fp64():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(200, D, generator=g, dtype=torch.float64)
    w = 1 + 0.1 * torch.randn(D, generator=g, dtype=torch.float64)
    ref = w * x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6)
    got = onr.rms_norm(x.float(), w.float(), 1e-6).double()
    assert (got - ref).abs().max() < 1e-5
    x16, w16 = x.to(torch.bfloat16), w.to(torch.bfloat16)
    got16 = onr.rms_norm(x16, w16, 1e-6).double()
    x64, w64 = x16.double(), w16.double()
    ref16 = w64 * x64 / torch.sqrt((x64 * x64).mean(-1, keepdim=True) + 1e-6)
    # two bf16 roundings (after the normalisation and after the weight), unit roundoff 2^-8 each
    assert ((got16 - ref16).abs() / ref16.abs()).max() <= 2 * 2**-8 + 2**-16


def test_rope_closed_forms_fp64():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, 4, 1, D, generator=g, dtype=torch.float64)

    def rot(v, p):
        c, s = onr.rope_cos_sin(torch.tensor([[p]]), D, 1e6, torch.float64)
        return onr.apply_rotary_pos_emb(v, v, c, s)[0]

    # position 0 is the identity
    assert torch.equal(rot(x, 0), x)
    # The angles are fp32 (HF computes inv_freq * pos in fp32 whatever the model
    # dtype), so the checks below allow the fp32 angle error, ~pos * 2^-24 rad.
    # Each (i, i + D/2) pair keeps its norm: cos^2 + sin^2 = 1 to fp32 rounding.
    y = rot(x, 12345)
    n_in = x[..., : D // 2] ** 2 + x[..., D // 2 :] ** 2
    n_out = y[..., : D // 2] ** 2 + y[..., D // 2 :] ** 2
    assert ((n_in - n_out).abs() / n_in).max() < 1e-6
    # rotations compose: R(a) R(b) = R(a + b)
    assert (rot(rot(x, 700), 300) - rot(x, 1000)).abs().max() < 1e-3
    # pair i turns by pos * theta^(-2i/D)
    for i in (0, 5, 63):
        ang = 777 * 1e6 ** (-2 * i / D)
        z = rot(x, 777)
        want = x[0, 0, 0, i] * math.cos(ang) - x[0, 0, 0, i + D // 2] * math.sin(ang)
        assert abs(float(z[0, 0, 0, i]) - float(want)) < 1e-4 * (1 + abs(float(want)))


def _sumsq_kernel_order(sq: np.ndarray) -> np.ndarray:
    """The order the HIP kernel sums squares in (see the module docstring)."""
    n = sq.shape[1]
    acc = [np.zeros(sq.shape[0], np.float32) for _ in range(32)]  # acc[k*8 + l]
    for i in range(0, n, 32):
        for k in range(4):
            for l in range(8):
                acc[k * 8 + l] = (acc[k * 8 + l] + sq[:, i + 8 * k + l]).astype(np.float32)
    total = np.zeros(sq.shape[0], np.float32)
    for l in range(8):
        v = acc[l]
        for k in range(1, 4):
            v = (v + acc[k * 8 + l]).astype(np.float32)
        total = (total + v).astype(np.float32)
    return total


@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_cpu_mean_square_order(head_dim):
    g = torch.Generator().manual_seed(head_dim)
    x = (torch.randn(20000, head_dim, generator=g) * torch.rand(20000, 1, generator=g) * 5).float()
    torch_mean = x.pow(2).mean(-1).numpy()
    mine = _sumsq_kernel_order((x * x).numpy()) / np.float32(head_dim)
    assert np.array_equal(mine, torch_mean)
