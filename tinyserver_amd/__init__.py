"""tinyserver_amd: the Qwen3 attention hot path of tinyserver on MI355X (gfx950).

Four hand-written HIP kernels behind a C ABI (include/tsa_api.h, libtsa.so):
fused QK RMSNorm + RoPE, the paged K/V store, paged GQA decode attention and
varlen causal prefill. ``tinyserver_amd.kernels`` mirrors the reference's
kernel modules; ``tinyserver_amd.patches.qwen3`` mirrors its Qwen3 attention
patch.
"""

__version__ = "0.1.0"
