"""QK RMSNorm + rotate-half RoPE, restated on the CPU (test infrastructure).

The arithmetic lives in the third-party ``transformers`` package that the
reference imports (server/model/patches/qwen3.py:11, called at :268-287).
Pinned version: transformers 5.15.0, file models/qwen3/modeling_qwen3.py.
Every rounding point is kept where that code has it, because one bf16 flip at
|x| in [4, 8) is already 0.031:

* RMSNorm (modeling_qwen3.py:59-64): x -> fp32; var = mean(x^2) in fp32;
  y = x * rsqrt(var + eps) in fp32; y -> model dtype; out = weight * y in the
  model dtype (one rounding of the exact product).
* cos/sin (modeling_qwen3.py:116-137): inv_freq = 1 / theta^(arange(0,D,2)/D)
  in fp32; freqs = inv_freq * pos in fp32; emb = cat(freqs, freqs);
  cos/sin in fp32, then cast to the model dtype.
* apply_rotary_pos_emb (modeling_qwen3.py:140-170): q*cos and
  rotate_half(q)*sin each round to the model dtype, then their sum rounds.
"""

from __future__ import annotations

import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Qwen3RMSNorm.forward (transformers modeling_qwen3.py:59-64)."""
    input_dtype = x.dtype
    h = x.to(torch.float32)
    variance = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(variance + eps)
    return weight * h.to(input_dtype)


def rope_inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """compute_default_rope_parameters (modeling_qwen3.py:116-122), fp32."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))


def rope_cos_sin(
    position_ids: torch.Tensor, head_dim: int, theta: float, dtype: torch.dtype
) -> tuple[torch.Tensor, torch.Tensor]:
    """Qwen3RotaryEmbedding.forward (modeling_qwen3.py:124-137).

    position_ids: (batch, T) integer. Returns cos, sin of shape (batch, T, D)
    in ``dtype``; the angles and trig are fp32 and round once at the end.
    """
    inv_freq = rope_inv_freq(head_dim, theta)
    inv_freq_expanded = inv_freq[None, :, None].float().expand(position_ids.shape[0], -1, 1)
    position_ids_expanded = position_ids[:, None, :].float()
    freqs = (inv_freq_expanded.float() @ position_ids_expanded.float()).transpose(1, 2)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """rotate_half (modeling_qwen3.py:140-144): cat(-x2, x1)."""
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2 :]
    return torch.cat((-x2, x1), dim=-1)


def apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim: int = 1):
    """apply_rotary_pos_emb (modeling_qwen3.py:148-170)."""
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    q_embed = (q * cos) + (rotate_half(q) * sin)
    k_embed = (k * cos) + (rotate_half(k) * sin)
    return q_embed, k_embed


def qk_norm_rope(
    q: torch.Tensor,
    k: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The call-site sequence of server/model/patches/qwen3.py:264-287.

    q: (1, T, Hq, D), k: (1, T, Hkv, D) -- the head-split projection outputs.
    cos, sin: (1, T, D). Returns the rotated q (1, Hq, T, D) and k
    (1, Hkv, T, D), exactly the tensors the reference hands to the store and
    to attention.
    """
    q = rms_norm(q, q_weight, eps)  # qwen3.py:268-269
    k = rms_norm(k, k_weight, eps)  # qwen3.py:270-271
    q = q.transpose(1, 2)  # qwen3.py:273
    k = k.transpose(1, 2)  # qwen3.py:274
    return apply_rotary_pos_emb(q, k, cos, sin)  # qwen3.py:287
