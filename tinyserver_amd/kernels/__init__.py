"""Drop-in replacements for tinyserver's Triton kernel modules.

Same module names, function names, signatures and ValueError guards as
server/model/kernels/{kv_cache,paged_attention,varlen_attention}.py, backed by
the gfx950 HIP library; plus the fused QK RMSNorm + RoPE the reference runs as
eager PyTorch, the batched sampler of server/model/sampling.py, and a
continuous-batching step's prefill and decode attention in one launch.
"""

from .kv_cache import store_kv_cache, store_kv_cache_batched, store_kv_cache_paged
from .mixed_attention import mixed_attention
from .paged_attention import paged_attention_forward, paged_decode_step
from .qk_norm_rope import qk_norm_rope, qk_norm_rope_store
from .sampling import sample_tokens
from .varlen_attention import flash_attn_varlen_func

__all__ = [
    "store_kv_cache",
    "store_kv_cache_batched",
    "store_kv_cache_paged",
    "paged_attention_forward",
    "paged_decode_step",
    "flash_attn_varlen_func",
    "qk_norm_rope",
    "qk_norm_rope_store",
    "sample_tokens",
    "mixed_attention",
]
