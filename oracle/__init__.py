"""CPU oracle for the Qwen3 attention hot path of tinyserver.

TEST INFRASTRUCTURE ONLY. This package restates, op for op on the CPU in
PyTorch, what the reference computes on this path. It is what the HIP kernels
are compared against in the tests, and the CPU baseline that bench.py times
beside them. Only ``tests/``, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline
leg may import it. The product path (``tinyserver_amd``) never imports it and
has no CPU fallback: without the HIP library it raises.

Modules
-------
norm_rope   QK RMSNorm and rotate-half RoPE, restating the third-party HF
            Qwen3 code the reference calls (transformers 5.15.0,
            models/qwen3/modeling_qwen3.py:59-64, 116-137, 140-170).
kv_store    The paged K/V stores (server/model/kernels/kv_cache.py) and their
            inverse gather (server/model/patches/qwen3.py:423-466).
paged       Paged decode attention (server/model/kernels/paged_attention.py)
            and the reference's CPU decode branch (patches/qwen3.py:359-385).
varlen      Varlen causal prefill (server/model/kernels/varlen_attention.py)
            and the reference's CPU prefill branch (patches/qwen3.py:132-171).
sampling    The batched sampler (server/model/sampling.py:119-194), the
            reference test's allowed-set rule, and a decision-margin helper.

How each function is pinned (known answers, closed forms, transformers on the
CPU, the reference tests' own cases) is listed in the tests that check it:
tests/test_oracle_*.py. No function here is unpinned.
"""

from . import kv_store, norm_rope, paged, sampling, varlen  # noqa: F401
