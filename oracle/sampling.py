"""Batched token sampling, restated on the CPU (test infrastructure).

* ``sample_tokens`` -- the reference's batched sampler
  (server/model/sampling.py:119-194): per-row temperature scaling in fp32,
  stable descending sort, top-k mask at rank >= k, softmax, top-p removal of
  the ranks whose preceding mass exceeds top_p (rank 0 kept), inverse-CDF pick
  with searchsorted (first rank whose cdf >= u * total), greedy rows (T <= 0)
  take rank 0. The same torch ops in the same order, in fp32, on the CPU.
* ``allowed_set`` -- the reference test's independent rule
  (tests/model/test_batch_sampling.py:27-52): a plain loop over the sorted
  order in fp64 giving every token that may legally be picked.
* ``decision_margin`` -- how close, in fp64, a row's decisions lie to their
  thresholds (the top-p cut and the pick). Implementations that sum the same
  fp32 masses in a different order may disagree only where this margin is
  within fp32 rounding.

Pinned by the reference tests' known answers (hand-computed CDF, greedy ties,
u = 0, per-row top-k, tiny top-p), by the allowed-set rule, and by the
closed-form pick frequencies over a grid of uniforms (tests/test_oracle_sampling.py).
"""

from __future__ import annotations

import torch

LOWEST_TEMPERATURE = 1e-5  # sampling.py:5


def sample_tokens(logits, temperature, top_k, top_p, uniforms, dtype=torch.float32):
    """sample_tokens (sampling.py:119-194) on the CPU, in fp32 as the
    reference computes; dtype=torch.float64 gives the same steps in fp64
    (closer to exact sums, for rows whose fp32 cumsum rounding is coarse)."""
    if logits.ndim != 2:
        raise ValueError(f"Expected logits shape [B, vocab_size], got {logits.ndim}D")
    batch_size, vocab_size = logits.shape
    for name, t in (("temperature", temperature), ("top_k", top_k), ("top_p", top_p), ("uniforms", uniforms)):
        if t.shape != (batch_size,):
            raise ValueError(f"Expected {name} shape [{batch_size}], got {tuple(t.shape)}")
    x = logits.float() / temperature.float().clamp(min=LOWEST_TEMPERATURE).unsqueeze(-1)
    x = x.to(dtype)
    sorted_x, order = torch.sort(x, dim=-1, descending=True, stable=True)
    ranks = torch.arange(vocab_size, device=logits.device).unsqueeze(0)
    k_eff = torch.where(top_k > 0, top_k, vocab_size).unsqueeze(-1)
    sorted_x = sorted_x.masked_fill(ranks >= k_eff, float("-inf"))
    probs = torch.softmax(sorted_x, dim=-1)
    cum = torch.cumsum(probs, dim=-1)
    remove = (cum - probs) > top_p.to(dtype).unsqueeze(-1)
    remove[:, 0] = False
    probs = probs.masked_fill(remove, 0.0)
    cdf = torch.cumsum(probs, dim=-1)
    targets = (uniforms.float().to(dtype).unsqueeze(-1) * cdf[:, -1:]).contiguous()
    picked = torch.searchsorted(cdf.contiguous(), targets).clamp(max=vocab_size - 1)
    rank = torch.where(temperature.unsqueeze(-1) <= 0, torch.zeros_like(picked), picked)
    return order.gather(-1, rank).squeeze(-1)


def _sorted_row(row, temperature):
    x = row.double() / max(float(temperature), LOWEST_TEMPERATURE)
    order = sorted(range(len(x)), key=lambda i: (-x[i].item(), i))
    return x, order


def allowed_set(row, temperature, top_k, top_p):
    """Tokens that may be picked (test_batch_sampling.py:27-52), fp64."""
    x, order = _sorted_row(row, temperature)
    if top_k > 0:
        order = order[:top_k]
    probs = torch.softmax(torch.tensor([x[i].item() for i in order], dtype=torch.float64), dim=-1)
    allowed, before = set(), 0.0
    for rank, token in enumerate(order):
        if rank == 0 or before <= top_p:
            allowed.add(token)
        before += probs[rank].item()
    return allowed


def decision_margin(row, temperature, top_k, top_p, uniform):
    """Smallest distance, in fp64 probability units, between a cumulative sum
    the row's decisions compare and the threshold it is compared with: the
    top-p test (mass before each rank vs top_p) around the cut, and the pick
    (cdf vs u * kept mass) around the picked rank. Greedy rows: +inf."""
    if temperature <= 0:
        return float("inf")
    x = row.double() / max(float(temperature), LOWEST_TEMPERATURE)
    xs, order = torch.sort(x, descending=True, stable=True)
    n = len(xs) if top_k <= 0 else min(top_k, len(xs))
    p = torch.softmax(xs[:n], dim=-1)
    cum = torch.cumsum(p, dim=0)
    before = cum - p
    keep = before <= top_p
    keep[0] = True
    last = int(keep.nonzero().max())  # kept ranks are 0..last
    margin = float("inf")
    if last >= 1:  # rank `last` kept: before[last] <= top_p
        margin = min(margin, abs(float(before[last]) - top_p))
    if last + 1 < n:  # rank `last + 1` removed: before[last + 1] > top_p
        margin = min(margin, abs(float(before[last + 1]) - top_p))
    kept = p[: last + 1]
    cdf = torch.cumsum(kept, dim=0)
    target = float(uniform) * float(cdf[-1])
    r = int(torch.searchsorted(cdf, torch.tensor([target], dtype=torch.float64)).clamp(max=last))
    margin = min(margin, abs(float(cdf[r]) - target))
    if r > 0:
        margin = min(margin, abs(float(cdf[r - 1]) - target))
    return margin
