"""The HIP path against the committed golden fixtures (tests/golden/), which
the CPU oracle wrote from seeded inputs: the stores bit-exact, norm/RoPE and
attention within max-abs 2e-2 / mean-abs 2e-3 (bf16, fp32 accumulation)."""

from pathlib import Path

import pytest
import torch
from safetensors.torch import load_file

from tests.helpers import assert_bitexact, assert_close
from tinyserver_amd.kernels import (flash_attn_varlen_func, paged_attention_forward, qk_norm_rope,
                                    store_kv_cache, store_kv_cache_batched)

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return {k: v.to(DEV) for k, v in load_file(str(GOLDEN / f"{name}.safetensors")).items()}


def test_norm_rope_golden():
    d = _load("norm_rope")
    qo, ko = qk_norm_rope(d["q"], d["k"], d["q_weight"], d["k_weight"], d["cos"], d["sin"], float(d["eps"][0]))
    torch.cuda.synchronize()
    assert_close(qo, d["q_out"], what="q golden")
    assert_close(ko, d["k_out"], what="k golden")
    same = (torch.eq(qo, d["q_out"]).float().mean() + torch.eq(ko, d["k_out"]).float().mean()) / 2
    assert same.item() >= 0.999


def test_store_golden():
    d = _load("store")
    kc, vc = d["k_cache"].clone(), d["v_cache"].clone()
    store_kv_cache(int(d["start"][0]), d["block_table"], d["k1"], d["v1"], kc, vc)
    store_kv_cache_batched(d["k2"], d["v2"], kc, vc, d["block_mapping"], d["slot_mapping"])
    torch.cuda.synchronize()
    assert_bitexact(kc, d["k_cache_out"])
    assert_bitexact(vc, d["v_cache_out"])


def test_paged_decode_golden():
    d = _load("paged_decode")
    out = paged_attention_forward(d["query"], d["k_cache"], d["v_cache"], d["block_tables"], 16, d["seq_lens"])
    torch.cuda.synchronize()
    assert_close(out, d["out"], what="decode golden")


def test_varlen_prefill_golden():
    d = _load("varlen_prefill")
    cu = d["cu_seqlens"]
    out = flash_attn_varlen_func(d["q"], d["k"], d["v"], cu, cu, 40, 40, True)
    torch.cuda.synchronize()
    assert_close(out, d["out"], what="prefill golden")
