"""Fused QK RMSNorm + RoPE (+ paged store) on the GPU vs the oracle.

The oracle follows HF's rounding points op for op (transformers
modeling_qwen3.py:59-64, 148-170). The kernel keeps the same rounding points;
only the fp32 order of the 128-term sum of squares differs, which can move a
rounded value by one bf16 ulp in rare cases. Tolerance: max-abs 2e-2,
mean-abs 2e-3, and at most 1 in 10^4 elements not bit-identical. The fused
store must write exactly the kernel's own rotated K and the raw V
(bit-exact), through the block tables.
"""

import pytest
import torch

from oracle import kv_store as ok
from oracle import norm_rope as onr
from tests.helpers import assert_bitexact, assert_close
from tinyserver_amd import workloads as W
from tinyserver_amd.kernels import qk_norm_rope, qk_norm_rope_store

pytestmark = pytest.mark.gpu
DEV = "cuda"
MAX_MISMATCH = 1e-4


def _oracle(q, k, w):
    """q (T, Hq, D), k (T, Hkv, D) -> rotated (T, H, D) through the call-site sequence."""
    qr, kr = onr.qk_norm_rope(q[None], k[None], w.q_weight, w.k_weight, w.cos[None], w.sin[None], w.eps)
    return qr[0].transpose(0, 1), kr[0].transpose(0, 1)


def _check(got, ref, what):
    assert_close(got, ref, what=what)
    same = (got.cpu() == ref).float().mean().item()
    print(f"{what}: bit-identical fraction {same:.6f}", flush=True)
    assert 1 - same <= MAX_MISMATCH, f"{what}: {1 - same:.2e} of elements differ"


@pytest.mark.parametrize("name", ["qwen3-0.6b-decode-bs4", "qwen3-8b-decode-bs64", "qwen3-8b-prefill-16seq"])
def test_matches_oracle(name):
    w = W.make(name)
    qr, kr = _oracle(w.q, w.k, w)
    qg, kg = qk_norm_rope(w.q.to(DEV), w.k.to(DEV), w.q_weight.to(DEV), w.k_weight.to(DEV), w.cos.to(DEV),
                          w.sin.to(DEV), w.eps)
    torch.cuda.synchronize()
    _check(qg, qr, f"{name} q")
    _check(kg, kr, f"{name} k")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_other_dtypes(dtype, head_dim):
    w = W.make_prefill("small", 11, 3, 8, 2, 5, 40, dtype=dtype, head_dim=head_dim)
    qr, kr = _oracle(w.q, w.k, w)
    qg, kg = qk_norm_rope(w.q.to(DEV), w.k.to(DEV), w.q_weight.to(DEV), w.k_weight.to(DEV), w.cos.to(DEV),
                          w.sin.to(DEV), w.eps)
    torch.cuda.synchronize()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert_close(qg, qr, max_abs=tol, mean_abs=tol / 10, what=f"{dtype} q")
    assert_close(kg, kr, max_abs=tol, mean_abs=tol / 10, what=f"{dtype} k")


def test_strided_projection_views():
    """q/k as views of one fused projection output (1, T, (Hq+2Hkv)*D)."""
    w = W.make("qwen3-4b-prefill-8seq")
    T, hq, hkv, d = w.q.shape[0], w.q.shape[1], w.k.shape[1], w.q.shape[2]
    fused = torch.cat([w.q.reshape(T, -1), w.k.reshape(T, -1), w.v.reshape(T, -1)], dim=1).to(DEV)
    q = fused[:, : hq * d].view(T, hq, d)
    k = fused[:, hq * d : (hq + hkv) * d].view(T, hkv, d)
    qr, kr = _oracle(w.q, w.k, w)
    qg, kg = qk_norm_rope(q, k, w.q_weight.to(DEV), w.k_weight.to(DEV), w.cos.to(DEV), w.sin.to(DEV), w.eps)
    torch.cuda.synchronize()
    _check(qg, qr, "q")
    _check(kg, kr, "k")


@pytest.mark.parametrize("mode", ["decode", "prefill"])
def test_fused_store(mode):
    if mode == "decode":
        w = W.make("qwen3-0.6b-decode-bs4", poison=True)
        b = len(w.ctx_lens)
        cu = torch.arange(b + 1, dtype=torch.int32)
        pos = w.positions
    else:
        w = W.make("qwen3-4b-prefill-8seq", poison=True)
        cu, pos = w.cu_seqlens, None
    _store_and_check(w, cu, pos)


# Head layouts around the 8-lanes-per-row kernel's edges (a token's H rows
# on 8*H lanes in whole waves): waves holding both q and k rows (Hq not a
# multiple of 8), dead lanes in the last wave (H not a multiple of 8), the
# 32B shape (9 waves), H = 128 (1024 lanes, the largest it takes) and
# H = 136 (past it: the per-row kernel).
@pytest.mark.parametrize("hq,hkv", [(6, 2), (12, 4), (5, 1), (40, 8), (64, 8), (120, 8), (128, 8)])
def test_fused_store_head_layouts(hq, hkv):
    w = W.make_prefill("heads", 12, 3, hq, hkv, 5, 40, poison=True)
    _store_and_check(w, w.cu_seqlens, None)


def _store_and_check(w, cu, pos):
    kc, vc = w.k_cache.to(DEV), w.v_cache.to(DEV)
    qg, kg = qk_norm_rope_store(w.q.to(DEV), w.k.to(DEV), w.v.to(DEV), w.q_weight.to(DEV), w.k_weight.to(DEV),
                                w.cos.to(DEV), w.sin.to(DEV), w.eps, kc, vc, w.block_tables.to(DEV), cu.to(DEV),
                                None if pos is None else pos.to(DEV))
    torch.cuda.synchronize()
    qr, kr = _oracle(w.q, w.k, w)
    _check(qg, qr, "q")
    _check(kg, kr, "k")
    # The cache holds exactly the kernel's rotated K and the raw V.
    ke, ve = w.k_cache.clone(), w.v_cache.clone()
    cul = cu.tolist()
    for s, lst in enumerate(w.block_lists):
        p0 = 0 if pos is None else int(pos[s])
        sl = slice(cul[s], cul[s + 1])
        ok.store_kv_cache(p0, torch.tensor(lst), kg.cpu()[sl].transpose(0, 1), w.v[sl].transpose(0, 1), ke, ve)
    assert_bitexact(kc, ke, "k_cache")
    assert_bitexact(vc, ve, "v_cache")


def _repage(w, bs, seed):
    """The workload's sequences on a pool of bs-token pages: fresh shuffled
    block tables and a random pool (the contents before the store)."""
    g = torch.Generator().manual_seed(seed)
    ctx = [int(n) for n in (w.ctx_lens if hasattr(w, "ctx_lens") and w.ctx_lens is not None else w.seq_lens)]
    npages = [max(1, -(-n // bs)) for n in ctx]
    nb = sum(npages) + 2
    perm = torch.randperm(nb, generator=g)
    tables, lists, cur = torch.zeros(len(ctx), max(npages), dtype=torch.int32), [], 0
    for i, n in enumerate(npages):
        lst = perm[cur:cur + n].tolist()
        tables[i, :n] = torch.tensor(lst, dtype=torch.int32)
        lists.append(lst)
        cur += n
    hkv, d = w.k_cache.shape[1], w.k_cache.shape[3]
    kc = torch.randn(nb, hkv, bs, d, generator=g).to(w.k_cache.dtype)
    vc = torch.randn(nb, hkv, bs, d, generator=g).to(w.v_cache.dtype)
    return tables, lists, kc, vc


@pytest.mark.parametrize("mode", ["decode", "prefill"])
def test_fused_store_page_256(mode):
    """The fused norm/RoPE/store on 256-token pages (the server's default page size)."""
    if mode == "decode":
        w = W.make("qwen3-0.6b-decode-bs4", poison=True)
        b = len(w.ctx_lens)
        cu, pos = torch.arange(b + 1, dtype=torch.int32), w.positions
    else:
        w = W.make("qwen3-4b-prefill-8seq", poison=True)
        cu, pos = w.cu_seqlens, None
    tables, lists, kc0, vc0 = _repage(w, 256, seed=5)
    kc, vc = kc0.to(DEV), vc0.to(DEV)
    qg, kg = qk_norm_rope_store(w.q.to(DEV), w.k.to(DEV), w.v.to(DEV), w.q_weight.to(DEV), w.k_weight.to(DEV),
                                w.cos.to(DEV), w.sin.to(DEV), w.eps, kc, vc, tables.to(DEV), cu.to(DEV),
                                None if pos is None else pos.to(DEV))
    torch.cuda.synchronize()
    qr, kr = _oracle(w.q, w.k, w)
    _check(qg, qr, "q")
    _check(kg, kr, "k")
    ke, ve = kc0.clone(), vc0.clone()
    cul = cu.tolist()
    for s, lst in enumerate(lists):
        p0 = 0 if pos is None else int(pos[s])
        sl = slice(cul[s], cul[s + 1])
        ok.store_kv_cache(p0, torch.tensor(lst), kg.cpu()[sl].transpose(0, 1), w.v[sl].transpose(0, 1), ke, ve)
    assert_bitexact(kc, ke, "k_cache")
    assert_bitexact(vc, ve, "v_cache")
