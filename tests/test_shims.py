"""The Python drop-in functions keep the reference's guards and fail loudly.

The ValueErrors of server/model/kernels/{kv_cache,paged_attention,varlen_attention}.py
(tests/model/test_kv_cache_kernels.py:210-255, test_paged_attention_kernel.py:225-234)
are raised before anything touches a device; with well-formed CPU tensors the
functions raise instead of computing on the CPU -- there is no CPU fallback.
"""

import pytest
import torch

from tinyserver_amd.kernels import (flash_attn_varlen_func, paged_attention_forward, qk_norm_rope,
                                    store_kv_cache, store_kv_cache_batched, store_kv_cache_paged)


def test_store_batched_guards():
    kc = torch.zeros(2, 2, 4, 8)
    with pytest.raises(ValueError, match="3D"):
        store_kv_cache_batched(torch.zeros(2, 8), torch.zeros(2, 1, 8), kc, kc.clone(), torch.zeros(1, dtype=torch.int32),
                               torch.zeros(1, dtype=torch.int32))
    with pytest.raises(ValueError):
        store_kv_cache_batched(torch.zeros(2, 3, 8), torch.zeros(2, 4, 8), kc, kc.clone(),
                               torch.zeros(3, dtype=torch.int32), torch.zeros(3, dtype=torch.int32))
    with pytest.raises(ValueError):
        store_kv_cache_batched(torch.zeros(2, 4, 8), torch.zeros(2, 4, 8), kc, kc.clone(),
                               torch.zeros(3, dtype=torch.int32), torch.zeros(4, dtype=torch.int32))


def test_store_guards():
    kc = torch.zeros(2, 2, 4, 8)
    with pytest.raises(ValueError, match="3D"):
        store_kv_cache(0, torch.zeros(1, dtype=torch.int32), torch.zeros(2, 8), torch.zeros(2, 1, 8), kc, kc.clone())
    with pytest.raises(ValueError):
        store_kv_cache_paged(torch.zeros(2, 4, 8), torch.zeros(2, 4, 8), kc, kc.clone(),
                             torch.zeros(2, 1, dtype=torch.int32), torch.zeros(2, dtype=torch.int32))


def test_paged_attention_guard():
    with pytest.raises(ValueError, match="3D"):
        paged_attention_forward(torch.zeros(4, 64), torch.zeros(2, 4, 16, 64), torch.zeros(2, 4, 16, 64),
                                torch.zeros(1, 1, dtype=torch.int32), 16, torch.ones(1, dtype=torch.int32))
    with pytest.raises(ValueError, match="block_size"):
        paged_attention_forward(torch.zeros(1, 4, 64), torch.zeros(2, 4, 16, 64), torch.zeros(2, 4, 16, 64),
                                torch.zeros(1, 1, dtype=torch.int32), 8, torch.ones(1, dtype=torch.int32))


def test_varlen_guards():
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(ValueError, match="3D"):
        flash_attn_varlen_func(torch.zeros(4, 64), torch.zeros(4, 1, 64), torch.zeros(4, 1, 64), cu, cu, 4, 4, True)
    with pytest.raises(ValueError, match="divisible"):
        flash_attn_varlen_func(torch.zeros(4, 3, 64), torch.zeros(4, 2, 64), torch.zeros(4, 2, 64), cu, cu, 4, 4, True)


def test_no_cpu_fallback():
    """Well-formed CPU tensors raise -- the kernels run only on the GPU."""
    q = torch.zeros(1, 4, 64)
    kc = torch.zeros(2, 4, 16, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        paged_attention_forward(q, kc, kc.clone(), torch.zeros(1, 1, dtype=torch.int32), 16,
                                torch.ones(1, dtype=torch.int32))
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        flash_attn_varlen_func(torch.zeros(4, 4, 64), torch.zeros(4, 4, 64), torch.zeros(4, 4, 64), cu, cu, 4, 4, True)
    with pytest.raises(RuntimeError, match="GPU"):
        qk_norm_rope(torch.zeros(3, 4, 64), torch.zeros(3, 2, 64), torch.ones(64), torch.ones(64), torch.ones(3, 64),
                     torch.zeros(3, 64), 1e-6)
