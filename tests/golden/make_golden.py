"""Write the golden fixtures of this directory from the CPU oracle.

Each fixture holds the seeded inputs of one kernel function and the oracle's
output for them, small enough to commit (safetensors, loaded without code
execution). tests/test_golden.py checks that the oracle still reproduces
them; tests/test_gpu_golden.py checks the HIP path against them.

Run from the repository root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import torch
from safetensors.torch import save_file

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import kv_store as ok  # noqa: E402
from oracle import norm_rope as onr  # noqa: E402
from oracle import paged as op  # noqa: E402
from oracle import varlen as ov  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def norm_rope(seed=101):
    """QK RMSNorm + RoPE of 5 tokens at positions 0..4095 (Qwen3 eps/theta)."""
    g = torch.Generator().manual_seed(seed)
    T, hq, hkv, D = 5, 4, 2, 128
    q = torch.randn(T, hq, D, generator=g).mul(3.0).to(torch.bfloat16)
    k = torch.randn(T, hkv, D, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    pos = torch.tensor([[0, 1, 7, 300, 4095]])
    cos, sin = onr.rope_cos_sin(pos, D, 1e6, torch.bfloat16)
    qo, ko = onr.qk_norm_rope(q[None], k[None], qw, kw, cos, sin, 1e-6)  # (1, H, T, D)
    return {"q": q, "k": k, "q_weight": qw, "k_weight": kw, "cos": cos[0].contiguous(), "sin": sin[0].contiguous(),
            "positions": pos[0].to(torch.int32), "eps": torch.tensor([1e-6], dtype=torch.float64),
            "q_out": qo[0].transpose(0, 1).contiguous(), "k_out": ko[0].transpose(0, 1).contiguous()}


def store(seed=102):
    """store_kv_cache (start 13, 6 tokens) then store_kv_cache_batched (5 tokens) into a 6-page pool."""
    g = torch.Generator().manual_seed(seed)
    hkv, D, BS, NB = 2, 128, 4, 6
    kc = torch.randn(NB, hkv, BS, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(NB, hkv, BS, D, generator=g).to(torch.bfloat16)
    k1 = torch.randn(hkv, 6, D, generator=g).to(torch.bfloat16)
    v1 = torch.randn(hkv, 6, D, generator=g).to(torch.bfloat16)
    table = torch.tensor([5, 0, 3, 1, 4], dtype=torch.int32)
    k2 = torch.randn(hkv, 5, D, generator=g).to(torch.bfloat16)
    v2 = torch.randn(hkv, 5, D, generator=g).to(torch.bfloat16)
    bmap = torch.tensor([2, 2, 0, 5, 1], dtype=torch.int64)
    smap = torch.tensor([0, 3, 2, 1, 3], dtype=torch.int64)
    ko, vo = kc.clone(), vc.clone()
    ok.store_kv_cache(13, table, k1, v1, ko, vo)
    ok.store_kv_cache_batched(k2, v2, ko, vo, bmap, smap)
    return {"k_cache": kc, "v_cache": vc, "k1": k1, "v1": v1, "block_table": table,
            "start": torch.tensor([13], dtype=torch.int64), "k2": k2, "v2": v2, "block_mapping": bmap,
            "slot_mapping": smap, "k_cache_out": ko, "v_cache_out": vo}


def paged_decode(seed=103):
    """3 sequences (ctx 1, 17, 70), 8 q / 2 kv heads, page 16, shuffled 12-page pool."""
    g = torch.Generator().manual_seed(seed)
    hq, hkv, D, BS, NB = 8, 2, 128, 16, 12
    ctx = [1, 17, 70]
    perm = torch.randperm(NB, generator=g).tolist()
    tables, nxt = [], 0
    for n in ctx:
        nb = -(-n // BS)
        tables.append(perm[nxt:nxt + nb])
        nxt += nb
    bt = torch.zeros(len(ctx), max(len(t) for t in tables), dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    kc = torch.randn(NB, hkv, BS, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(NB, hkv, BS, D, generator=g).to(torch.bfloat16)
    q = torch.randn(len(ctx), hq, D, generator=g).to(torch.bfloat16)
    sl = torch.tensor(ctx, dtype=torch.int32)
    out = op.paged_attention_forward(q, kc, vc, bt, BS, sl)
    return {"query": q, "k_cache": kc, "v_cache": vc, "block_tables": bt, "seq_lens": sl, "out": out.contiguous()}


def varlen_prefill(seed=104):
    """Causal varlen prefill of 3 packed sequences (1, 33, 40), 4 q / 2 kv heads, D 128."""
    g = torch.Generator().manual_seed(seed)
    lens = [1, 33, 40]
    T, hq, hkv, D = sum(lens), 4, 2, 128
    q = torch.randn(T, hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(T, hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(T, hkv, D, generator=g).to(torch.bfloat16)
    cu = torch.tensor([0, 1, 34, 74], dtype=torch.int32)
    out = ov.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), True)
    return {"q": q, "k": k, "v": v, "cu_seqlens": cu, "out": out.contiguous()}


FIXTURES = {"norm_rope": norm_rope, "store": store, "paged_decode": paged_decode, "varlen_prefill": varlen_prefill}


def main():
    torch.set_num_threads(1)
    for name, fn in FIXTURES.items():
        t = {k: v.contiguous() for k, v in fn().items()}
        path = os.path.join(HERE, f"{name}.safetensors")
        save_file(t, path)
        print(f"{path}: {sum(v.numel() * v.element_size() for v in t.values())} bytes")


if __name__ == "__main__":
    main()
