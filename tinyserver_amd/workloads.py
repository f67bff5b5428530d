"""Seeded synthetic inputs for the attention path at the standard shapes.

One ``torch.Generator`` seed per workload; draw order is fixed: context
lengths -> page permutation -> cache contents -> new q/k/v -> norm weights.
Shapes follow Qwen3 attention (head_dim 128, page 16):

  qwen3-0.6b-decode-bs4     B=4,   16/8 heads, ctx U[16,512],   pool 256 pages
  qwen3-8b-decode-bs64      B=64,  32/8 heads, ctx U[512,4096], pool sum(pages)*1.1
  qwen3-8b-prefill-16seq    16 packed seqs, L U[128,2048], 32/8 heads
  qwen3-32b-decode-bs32     B=32,  64/8 heads, ctx 32768 each
  qwen3-4b-prefill-8seq     8 packed seqs, L U[256,1024], 32/8 heads
  qwen3-4b-mixed            one continuous-batching step on one shared pool:
                            8 new prefill seqs L U[256,1024], then 120 decode
                            seqs ctx U[256,8192]; 32/8 heads
  qwen3-4b-mixed-chunk      the same decode batch beside 2 short prefill
                            chunks, L U[128,512] (a chunked-prefill step)

A decode step stores one new token per sequence at position ctx-1 (pages for
positions 0..ctx-2 hold N(0,1) K/V) and attends over ctx tokens. cos/sin are
computed by transformers' Qwen3RotaryEmbedding, the code the model calls.
With ``poison`` the slots the step must not read (past ctx in the last page,
free pages, and the slot the step is about to write) hold 1e4.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

HEAD_DIM = 128
PAGE = 16
ROPE_THETA = 1.0e6
RMS_EPS = 1e-6


@dataclass
class DecodeWorkload:
    name: str
    seed: int
    ctx_lens: torch.Tensor       # (B,) int64, tokens attended after the store
    block_tables: torch.Tensor   # (B, max_blocks) int32, zero padded
    block_lists: list            # per-sequence lists (the InferenceContext form)
    k_cache: torch.Tensor        # (NB, Hkv, BS, D)
    v_cache: torch.Tensor
    q: torch.Tensor              # (B, Hq, D) raw projection of the new token
    k: torch.Tensor              # (B, Hkv, D)
    v: torch.Tensor              # (B, Hkv, D)
    q_weight: torch.Tensor       # (D,)
    k_weight: torch.Tensor
    cos: torch.Tensor            # (B, D) at position ctx-1
    sin: torch.Tensor
    eps: float = RMS_EPS

    @property
    def positions(self) -> torch.Tensor:
        return self.ctx_lens - 1

    @property
    def num_heads(self) -> int:
        return self.q.shape[1]

    @property
    def num_kv_heads(self) -> int:
        return self.k.shape[1]

    def to(self, device) -> "DecodeWorkload":
        kw = {f: getattr(self, f) for f in self.__dataclass_fields__}
        for f, val in kw.items():
            if isinstance(val, torch.Tensor):
                kw[f] = val.to(device)
        return DecodeWorkload(**kw)


@dataclass
class PrefillWorkload:
    name: str
    seed: int
    seq_lens: torch.Tensor       # (S,) int64
    cu_seqlens: torch.Tensor     # (S+1,) int32
    block_tables: torch.Tensor   # (S, max_blocks) int32
    block_lists: list
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    q: torch.Tensor              # (T, Hq, D) raw projections
    k: torch.Tensor              # (T, Hkv, D)
    v: torch.Tensor
    q_weight: torch.Tensor
    k_weight: torch.Tensor
    cos: torch.Tensor            # (T, D), positions 0..L-1 per sequence
    sin: torch.Tensor
    positions: torch.Tensor = field(default=None)
    eps: float = RMS_EPS

    @property
    def max_seqlen(self) -> int:
        return int(self.seq_lens.max())

    def to(self, device) -> "PrefillWorkload":
        kw = {f: getattr(self, f) for f in self.__dataclass_fields__}
        for f, val in kw.items():
            if isinstance(val, torch.Tensor):
                kw[f] = val.to(device)
        return PrefillWorkload(**kw)


def rope_cos_sin(positions: torch.Tensor, head_dim: int, theta: float, dtype: torch.dtype):
    """cos/sin as the model computes them (transformers Qwen3RotaryEmbedding)."""
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    cfg = Qwen3Config(head_dim=head_dim, hidden_size=head_dim * 8, num_attention_heads=8, num_key_value_heads=8,
                      rope_theta=theta, max_position_embeddings=1 << 20)
    rot = Qwen3RotaryEmbedding(cfg)
    dummy = torch.empty(0, dtype=dtype)
    cos, sin = rot(dummy, positions.reshape(1, -1).to(torch.int64).cpu())
    return cos[0], sin[0]


def _randn(gen, shape, dtype, device):
    return torch.randn(*shape, generator=gen, device=device, dtype=torch.float32).to(dtype)


def _assign_pages(gen, pages_per_seq: list[int], num_blocks: int, device):
    perm = torch.randperm(num_blocks, generator=gen, device=device).cpu()
    lists, cur = [], 0
    for n in pages_per_seq:
        lists.append([int(x) for x in perm[cur : cur + n]])
        cur += n
    max_blocks = max(max(pages_per_seq), 1)
    bt = torch.zeros(len(pages_per_seq), max_blocks, dtype=torch.int32)
    for i, lst in enumerate(lists):
        bt[i, : len(lst)] = torch.tensor(lst, dtype=torch.int32)
    return bt, lists


def _poison_unused(k_cache, v_cache, block_lists, used_lens):
    """1e4 everywhere except positions [0, used_len) of each sequence."""
    keep = torch.zeros(k_cache.shape[0], k_cache.shape[2], dtype=torch.bool, device=k_cache.device)
    for lst, n in zip(block_lists, used_lens):
        for j, blk in enumerate(lst):
            lo = j * k_cache.shape[2]
            cnt = max(0, min(k_cache.shape[2], int(n) - lo))
            keep[blk, :cnt] = True
    mask = (~keep)[:, None, :, None].expand_as(k_cache)
    k_cache[mask] = 1e4
    v_cache[mask] = 1e4


def make_decode(name, seed, batch, num_heads, num_kv_heads, ctx_lo, ctx_hi, num_blocks=None, pool_slack=1.1,
                dtype=torch.bfloat16, device="cpu", poison=False, head_dim=HEAD_DIM, page=PAGE, ctx_lens=None):
    gen = torch.Generator(device=device).manual_seed(seed)
    if ctx_lens is None:
        ctx = torch.randint(ctx_lo, ctx_hi + 1, (batch,), generator=gen, device=device).cpu()
    else:
        ctx = torch.as_tensor(ctx_lens, dtype=torch.int64)
    pages = [math.ceil(int(n) / page) for n in ctx]
    nb = num_blocks if num_blocks is not None else math.ceil(sum(pages) * pool_slack)
    if nb < sum(pages):
        raise ValueError(f"pool of {nb} pages cannot hold {sum(pages)}")
    bt, lists = _assign_pages(gen, pages, nb, device)
    k_cache = _randn(gen, (nb, num_kv_heads, page, head_dim), dtype, device)
    v_cache = _randn(gen, (nb, num_kv_heads, page, head_dim), dtype, device)
    q = _randn(gen, (batch, num_heads, head_dim), dtype, device)
    k = _randn(gen, (batch, num_kv_heads, head_dim), dtype, device)
    v = _randn(gen, (batch, num_kv_heads, head_dim), dtype, device)
    qw = (1.0 + 0.1 * torch.randn(head_dim, generator=gen, device=device)).to(dtype)
    kw = (1.0 + 0.1 * torch.randn(head_dim, generator=gen, device=device)).to(dtype)
    if poison:
        _poison_unused(k_cache, v_cache, lists, [int(n) - 1 for n in ctx])
    cos, sin = rope_cos_sin(ctx - 1, head_dim, ROPE_THETA, dtype)
    return DecodeWorkload(name, seed, ctx, bt.to(device), lists, k_cache, v_cache, q, k, v, qw, kw, cos.to(device),
                          sin.to(device))


def make_prefill(name, seed, num_seqs, num_heads, num_kv_heads, len_lo, len_hi, pool_slack=1.1,
                 dtype=torch.bfloat16, device="cpu", poison=False, head_dim=HEAD_DIM, page=PAGE, seq_lens=None):
    gen = torch.Generator(device=device).manual_seed(seed)
    if seq_lens is None:
        lens = torch.randint(len_lo, len_hi + 1, (num_seqs,), generator=gen, device=device).cpu()
    else:
        lens = torch.as_tensor(seq_lens, dtype=torch.int64)
    pages = [math.ceil(int(n) / page) for n in lens]
    nb = math.ceil(sum(pages) * pool_slack)
    bt, lists = _assign_pages(gen, pages, nb, device)
    k_cache = _randn(gen, (nb, num_kv_heads, page, head_dim), dtype, device)
    v_cache = _randn(gen, (nb, num_kv_heads, page, head_dim), dtype, device)
    T = int(lens.sum())
    q = _randn(gen, (T, num_heads, head_dim), dtype, device)
    k = _randn(gen, (T, num_kv_heads, head_dim), dtype, device)
    v = _randn(gen, (T, num_kv_heads, head_dim), dtype, device)
    qw = (1.0 + 0.1 * torch.randn(head_dim, generator=gen, device=device)).to(dtype)
    kw = (1.0 + 0.1 * torch.randn(head_dim, generator=gen, device=device)).to(dtype)
    if poison:
        _poison_unused(k_cache, v_cache, lists, [0] * len(lists))
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0).to(torch.int32)
    positions = torch.cat([torch.arange(int(n)) for n in lens]) if T else torch.zeros(0, dtype=torch.int64)
    cos, sin = rope_cos_sin(positions, head_dim, ROPE_THETA, dtype)
    return PrefillWorkload(name, seed, lens, cu.to(device), bt.to(device), lists, k_cache, v_cache, q, k, v, qw, kw,
                           cos.to(device), sin.to(device), positions.to(device))


# name -> (kind, kwargs). Seeds are fixed per workload.
WORKLOADS = {
    "qwen3-0.6b-decode-bs4": ("decode", dict(seed=1, batch=4, num_heads=16, num_kv_heads=8, ctx_lo=16, ctx_hi=512,
                                             num_blocks=256)),
    "qwen3-8b-decode-bs64": ("decode", dict(seed=2, batch=64, num_heads=32, num_kv_heads=8, ctx_lo=512, ctx_hi=4096)),
    "qwen3-8b-prefill-16seq": ("prefill", dict(seed=3, num_seqs=16, num_heads=32, num_kv_heads=8, len_lo=128,
                                               len_hi=2048)),
    "qwen3-32b-decode-bs32": ("decode", dict(seed=4, batch=32, num_heads=64, num_kv_heads=8, ctx_lo=32768,
                                             ctx_hi=32768, pool_slack=1.0)),
    # The mixed step's prefill shape on a pool of its own (a parity case for
    # the stores and the norm, which do not need the 2 GB shared pool).
    "qwen3-4b-prefill-8seq": ("prefill", dict(seed=6, num_seqs=8, num_heads=32, num_kv_heads=8, len_lo=256,
                                              len_hi=1024)),
    "qwen3-4b-mixed": ("mixed", dict(seed=5, decode_batch=120, ctx_lo=256, ctx_hi=8192, prefill_seqs=8,
                                     len_lo=256, len_hi=1024, num_heads=32, num_kv_heads=8)),
    "qwen3-4b-mixed-chunk": ("mixed", dict(seed=7, decode_batch=120, ctx_lo=256, ctx_hi=8192, prefill_seqs=2,
                                           len_lo=128, len_hi=512, num_heads=32, num_kv_heads=8)),
}


def make(name: str, **overrides):
    kind, kw = WORKLOADS[name]
    kw = {**kw, **overrides}
    maker = {"decode": make_decode, "prefill": make_prefill, "mixed": make_mixed}[kind]
    return maker(name, **kw)


@dataclass
class MixedWorkload:
    """One continuous-batching step over one shared KV pool, as the scheduler
    issues it: a prefill batch of new sequences, then a decode batch of the
    running ones (server/executor/scheduler.py:128-227; each batch is its own
    forward, server/model/patches/qwen3.py:291-327 then :328-416). The two
    halves own disjoint pages of the same k_cache/v_cache tensors and share
    the layer's norm weights."""

    name: str
    seed: int
    prefill: PrefillWorkload
    decode: DecodeWorkload

    @property
    def k_cache(self):
        return self.decode.k_cache

    @property
    def v_cache(self):
        return self.decode.v_cache

    def to(self, device) -> "MixedWorkload":
        d = self.decode.to(device)
        p = self.prefill.to(device)
        p.k_cache, p.v_cache = d.k_cache, d.v_cache  # still one pool
        return MixedWorkload(self.name, self.seed, p, d)


def make_mixed(name, seed, decode_batch, ctx_lo, ctx_hi, prefill_seqs, len_lo, len_hi, num_heads, num_kv_heads,
               pool_slack=1.1, dtype=torch.bfloat16, device="cpu", poison=False, head_dim=HEAD_DIM, page=PAGE):
    """The shared-pool step. Draw order: decode context lengths, prefill
    lengths, one page permutation of the pool (decode sequences take their
    pages first, then the prefill sequences), cache contents, decode q/k/v,
    prefill q/k/v, norm weights."""
    gen = torch.Generator(device=device).manual_seed(seed)
    ctx = torch.randint(ctx_lo, ctx_hi + 1, (decode_batch,), generator=gen, device=device).cpu()
    lens = torch.randint(len_lo, len_hi + 1, (prefill_seqs,), generator=gen, device=device).cpu()
    dpages = [math.ceil(int(n) / page) for n in ctx]
    ppages = [math.ceil(int(n) / page) for n in lens]
    nb = math.ceil((sum(dpages) + sum(ppages)) * pool_slack)
    bt_all, lists = _assign_pages(gen, dpages + ppages, nb, device)
    dlists, plists = lists[:decode_batch], lists[decode_batch:]
    dbt = bt_all[:decode_batch, : max(max(dpages), 1)].contiguous()
    pbt = bt_all[decode_batch:, : max(max(ppages), 1)].contiguous()
    k_cache = _randn(gen, (nb, num_kv_heads, page, head_dim), dtype, device)
    v_cache = _randn(gen, (nb, num_kv_heads, page, head_dim), dtype, device)
    dq = _randn(gen, (decode_batch, num_heads, head_dim), dtype, device)
    dk = _randn(gen, (decode_batch, num_kv_heads, head_dim), dtype, device)
    dv = _randn(gen, (decode_batch, num_kv_heads, head_dim), dtype, device)
    T = int(lens.sum())
    pq = _randn(gen, (T, num_heads, head_dim), dtype, device)
    pk = _randn(gen, (T, num_kv_heads, head_dim), dtype, device)
    pv = _randn(gen, (T, num_kv_heads, head_dim), dtype, device)
    qw = (1.0 + 0.1 * torch.randn(head_dim, generator=gen, device=device)).to(dtype)
    kw = (1.0 + 0.1 * torch.randn(head_dim, generator=gen, device=device)).to(dtype)
    if poison:  # everything but the decode sequences' stored prefixes
        _poison_unused(k_cache, v_cache, dlists + plists, [int(n) - 1 for n in ctx] + [0] * len(plists))
    dcos, dsin = rope_cos_sin(ctx - 1, head_dim, ROPE_THETA, dtype)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0).to(torch.int32)
    positions = torch.cat([torch.arange(int(n)) for n in lens])
    pcos, psin = rope_cos_sin(positions, head_dim, ROPE_THETA, dtype)
    dec = DecodeWorkload(name + ":decode", seed, ctx, dbt.to(device), dlists, k_cache, v_cache, dq, dk, dv, qw, kw,
                         dcos.to(device), dsin.to(device))
    pre = PrefillWorkload(name + ":prefill", seed, lens, cu.to(device), pbt.to(device), plists, k_cache, v_cache, pq,
                          pk, pv, qw, kw, pcos.to(device), psin.to(device), positions.to(device))
    return MixedWorkload(name, seed, pre, dec)


def decode_bytes(ctx_lens, num_heads, num_kv_heads, head_dim=HEAD_DIM, page=PAGE, elem=2) -> int:
    """Algorithmic HBM bytes of one paged decode attention call: every K/V
    byte once, q in, o out, the used block-table entries and seq_lens."""
    ctx = [int(n) for n in ctx_lens]
    b = len(ctx)
    kv = sum(ctx) * num_kv_heads * head_dim * elem * 2
    qo = 2 * b * num_heads * head_dim * elem
    tables = sum(math.ceil(n / page) for n in ctx) * 4 + 4 * b
    return kv + qo + tables


def prefill_flops(seq_lens, num_heads, head_dim=HEAD_DIM) -> int:
    """Causal QK^T + PV flops, diagonal included: 4 D Hq sum L(L+1)/2."""
    return sum(4 * head_dim * num_heads * int(n) * (int(n) + 1) // 2 for n in seq_lens)
