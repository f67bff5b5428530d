"""Paged-attention patch of HF Qwen3 on the gfx950 kernels (the call-site glue).

Mirrors server/model/patches/qwen3.py: the paged KV pool allocator (:21-64),
the per-layer attention forward (:67-418, ``_patch_single_layer`` /
``_page_attention_forward``), ``qwen3_model_patcher`` (:469-480) and
``qwen3_model_loader`` (:483-505). The model takes the reference's flattened
input: ``input_ids``/``position_ids`` of shape (1, total_tokens), and the
current ``InferenceContext`` saying whether the step is a prefill or a decode
and which pages each sequence owns. The context is read through the engine's
own getter, as the reference does (qwen3.py:14, :289): the patcher binds
``server.model.inference_context.get_inference_context`` when that module
imports, so the unchanged engine's ``with inference_context(ctx)`` is what
the layers see; without it, ``tinyserver_amd.inference_context`` (the same
contract) is used. Any object with ``mode`` and ``sequences`` works; nothing
is stored on it.

Per layer the reference runs q_norm, k_norm, apply_rotary_pos_emb and a store
loop (one launch per sequence at decode, a Python mapping loop at prefill),
then the attention kernel. Here one fused kernel does QK RMSNorm + RoPE +
the paged K/V store of every token (store before attend: the new token takes
part in attention), then varlen prefill or paged decode attention runs. The
metadata is built once per forward (the first layer builds it, the others
reuse it), not once per layer and per sequence: the block tables live on the
device (block_tables.BlockTableMirror) and a step uploads only the blocks
appended since the last one, with cu_seqlens, in one transfer.

Same errors as the reference: ValueError for prefill lengths that do not sum
to the flattened length or are not positive (:182-187) and for a missing
position_ids (:231-236, :329-330); MemoryError when not even one KV block
fits (:43-47). There is no CPU path: the kernels run on the GPU only, and
CPU tensors raise.
"""

from __future__ import annotations

import importlib
import weakref
from dataclasses import dataclass
from typing import Any, Callable

import numpy as np
import torch

from .. import inference_context as _own_context
from ..kernels import flash_attn_varlen_func, paged_attention_forward, paged_decode_step, qk_norm_rope_store
from .block_tables import BlockTableMirror

ENGINE_CONTEXT_MODULE = "server.model.inference_context"


def engine_context_getter() -> Callable[[], Any]:
    """The getter of the engine's current InferenceContext: the reference
    engine's module-global (server/model/inference_context.py:27-29) when that
    module imports, else this package's mirror of it."""
    try:
        return importlib.import_module(ENGINE_CONTEXT_MODULE).get_inference_context
    except ImportError:
        return _own_context.get_inference_context


def _available_memory(memory_utilization: float) -> int:
    """Free device memory times the utilisation, less the room the model's
    own peak use needs (server/model/utils.py:12-22)."""
    free, _ = torch.cuda.mem_get_info()
    stats = torch.cuda.memory_stats()
    reserve = stats.get("allocated_bytes.all.peak", 0) - stats.get("allocated_bytes.all.current", 0)
    return max(0, int(free * memory_utilization - reserve))


def qwen3_cache_allocator(model, config, memory_utilization: float, block_size: int, dtype: torch.dtype,
                          device: str) -> int:
    """Allocate the paged KV pool (2, layers, blocks, kv_heads, block_size,
    head_dim) and give every layer its K and V view. Returns the block count."""
    available = _available_memory(memory_utilization)
    elem = torch.tensor([], dtype=dtype).element_size()
    block_bytes = 2 * config.num_hidden_layers * block_size * config.num_key_value_heads * config.head_dim * elem
    num_blocks = int(available // block_bytes)
    if num_blocks <= 0:
        raise MemoryError(f"Not enough memory for even one block of KV cache: {available / 2**30:.2f} GB available, "
                          f"{block_bytes / 2**30:.2f} GB per block")
    pool = torch.zeros(2, config.num_hidden_layers, num_blocks, config.num_key_value_heads, block_size,
                       config.head_dim, device=device, dtype=dtype)
    for i, layer in enumerate(model.model.layers):
        layer.self_attn.k_cache = pool[0, i]
        layer.self_attn.v_cache = pool[1, i]
    return num_blocks


@dataclass
class DeviceMetadata:
    """What the kernels need to address the batch, on the device."""

    block_tables: torch.Tensor  # (B, max_blocks) int32, zero-padded
    cu_seqlens: torch.Tensor    # (B + 1,) int32 offsets into the flattened tokens
    max_seqlen: int
    positions: torch.Tensor | None  # decode: (B,) int32 position of each new token
    seq_lens: torch.Tensor | None   # decode: (B,) int32 = positions + 1
    table_slots: int = 0            # sum of the block tables' lengths (host-side size of the step's KV)


# The device-resident block tables, one mirror per device.
_mirrors: dict[torch.device, BlockTableMirror] = {}

# The last build: (weak reference to its context, position_ids, key, metadata).
# One entry suffices: the layers of a forward run one after another on the
# engine's single thread (the reference's own assumption for its context,
# server/model/inference_context.py:7-10).
_last_build: tuple | None = None


def device_metadata(ctx: Any, position_ids: torch.Tensor | None, num_tokens: int,
                    device: torch.device) -> DeviceMetadata:
    """Build the padded block tables, cu_seqlens and, for a decode step, the
    positions and sequence lengths, with the reference's checks. The block
    tables come from the device's BlockTableMirror, which uploads only the
    blocks appended since it last saw each sequence's list; cu_seqlens rides
    in the same transfer.

    ``ctx`` is any object with ``mode`` and ``sequences`` (the reference's
    InferenceContext, server/model/inference_context.py:18-21). The layers of
    one forward share the build: they see the same context object and the
    same position_ids tensor, which HF hands every layer; the engine makes a
    new context every step (server/executor/engine.py:579-582), and the
    cache holds only a weak reference to it, so a later step -- or a context
    at a recycled address -- never hits a stale entry. A context that cannot
    be weakly referenced is rebuilt per layer. The context's sequences must
    not be changed in place during a forward."""
    global _last_build
    key = (ctx.mode, num_tokens, str(device), getattr(position_ids, "_version", None))
    last = _last_build
    if last is not None and last[0]() is ctx and last[1] is position_ids and last[2] == key:
        return last[3]
    seqs = ctx.sequences
    if ctx.mode == "prefill":
        lengths = [int(s["num_tokens"]) for s in seqs]
        if sum(lengths) != num_tokens:
            raise ValueError(f"Prefill sequence lengths sum to {sum(lengths)}, expected flattened seq_len {num_tokens}")
        if any(n <= 0 for n in lengths):
            raise ValueError("Prefill sequence lengths must all be positive")
    else:
        if position_ids is None:
            raise ValueError("Position ids should not be None for decode attention")
        if len(seqs) != num_tokens:
            raise ValueError(f"Decode step has {num_tokens} tokens for {len(seqs)} sequences")
        lengths = [1] * len(seqs)
    tables = [s["block_table"] for s in seqs]
    cu = np.zeros(len(seqs) + 1, dtype=np.int64)
    np.cumsum(lengths, out=cu[1:])
    mirror = _mirrors.get(device)
    if mirror is None:
        mirror = _mirrors[device] = BlockTableMirror(device)
    block_tables, cu_seqlens = mirror.gather(tables, cu)
    positions = seq_lens = None
    if ctx.mode != "prefill":
        positions = position_ids.reshape(-1).to(device=device, dtype=torch.int32)
        seq_lens = positions + 1
    meta = DeviceMetadata(block_tables, cu_seqlens, max(lengths, default=0), positions, seq_lens,
                          sum(len(t) for t in tables))
    try:
        ref = weakref.ref(ctx)
    except TypeError:  # (e.g. a slotted class without __weakref__): no caching
        ref = None
    _last_build = (ref, position_ids, key, meta) if ref is not None else None
    return meta


# A decode step whose KV spans at most this many 16-token tiles (per kv head
# summed over the heads) takes the single-launch fused step; larger ones take
# the norm/store launch followed by paged attention. The fused kernel saves a
# launch (a few microseconds) but pays at every (sequence, kv head) unit it
# enters (the unit's loads into LDS, its norm, a wait for them), which
# outweighs the saved launch on large steps. Measured at head_dim 128 on 256
# CUs: Qwen3-0.6B batch 4 (550 tiles) 29 us fused vs 50 us; Qwen3-8B batch 64
# (74k tiles) 131 us vs 132 us; a 120-sequence batch (257k tiles) 394 us vs
# 357 us.
FUSED_DECODE_MAX_TILES = 16384


def _patch_single_layer(layer: torch.nn.Module,
                        rotary_emb: Callable[[torch.Tensor, torch.Tensor], tuple[torch.Tensor, torch.Tensor]],
                        get_context: Callable[[], Any]) -> None:
    """Replace layer.self_attn.forward by the paged forward on the kernels."""
    attn = layer.self_attn
    cfg = attn.config
    num_heads, num_kv_heads, head_dim = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    if not (hasattr(attn, "q_norm") and hasattr(attn, "k_norm")):
        raise NotImplementedError("the fused kernel applies Qwen3's QK RMSNorm; this attention module has none")

    def _page_attention_forward(hidden_states: torch.Tensor, attention_mask: torch.Tensor | None = None,
                                position_ids: torch.LongTensor | None = None, past_key_values=None,
                                use_cache: bool = False,
                                position_embeddings: tuple[torch.Tensor, torch.Tensor] | None = None, **kwargs):
        batch, seq_len, _ = hidden_states.shape  # batch is 1: the flattened step
        q = attn.q_proj(hidden_states).view(batch * seq_len, num_heads, head_dim)
        k = attn.k_proj(hidden_states).view(batch * seq_len, num_kv_heads, head_dim)
        v = attn.v_proj(hidden_states).view(batch * seq_len, num_kv_heads, head_dim)
        if position_embeddings is not None:
            cos, sin = position_embeddings
        else:
            if position_ids is None:
                raise ValueError("Position ids should not be None for the patched attention forward")
            cos, sin = rotary_emb(v, position_ids)
        cos = cos.reshape(-1, head_dim)
        sin = sin.reshape(-1, head_dim)

        ctx = get_context()
        meta = device_metadata(ctx, position_ids, batch * seq_len, hidden_states.device)
        block_size = attn.k_cache.shape[2]
        if ctx.mode == "prefill":
            q_rot, k_rot = qk_norm_rope_store(q, k, v, attn.q_norm.weight, attn.k_norm.weight, cos, sin,
                                              attn.q_norm.variance_epsilon, attn.k_cache, attn.v_cache,
                                              meta.block_tables, meta.cu_seqlens)
            out = flash_attn_varlen_func(q_rot, k_rot, v, meta.cu_seqlens, meta.cu_seqlens, meta.max_seqlen,
                                         meta.max_seqlen, causal=True, softmax_scale=head_dim**-0.5)
        elif (getattr(attn, "_tsa_fused_decode", True)
              and meta.table_slots * block_size // 16 * num_kv_heads <= FUSED_DECODE_MAX_TILES):
            try:
                out = paged_decode_step(q, k, v, attn.q_norm.weight, attn.k_norm.weight, cos, sin,
                                        attn.q_norm.variance_epsilon, attn.k_cache, attn.v_cache,
                                        meta.block_tables, meta.seq_lens)
            except NotImplementedError:  # a shape the fused kernel does not cover: stop trying it
                attn._tsa_fused_decode = False
                return _page_attention_forward(hidden_states, attention_mask, position_ids, past_key_values,
                                               use_cache, position_embeddings, **kwargs)
        else:
            q_rot, _ = qk_norm_rope_store(q, k, v, attn.q_norm.weight, attn.k_norm.weight, cos, sin,
                                          attn.q_norm.variance_epsilon, attn.k_cache, attn.v_cache,
                                          meta.block_tables, meta.cu_seqlens, meta.positions, return_k=False)
            out = paged_attention_forward(q_rot, attn.k_cache, attn.v_cache, meta.block_tables, block_size,
                                          meta.seq_lens)
        return attn.o_proj(out.reshape(batch, seq_len, num_heads * head_dim)), None

    attn.forward = _page_attention_forward


def qwen3_model_patcher(model, get_context: Callable[[], Any] | None = None):
    """Route every layer's attention through the paged kernels. The layers
    read the step's context through ``get_context`` (default: the engine's
    getter, ``engine_context_getter()``)."""
    getter = get_context if get_context is not None else engine_context_getter()
    for layer in model.model.layers:
        _patch_single_layer(layer, model.model.rotary_emb, getter)
    return model


def qwen3_model_loader(model, config, memory_utilization: float, block_size: int, dtype: torch.dtype,
                       device: str, get_context: Callable[[], Any] | None = None) -> int:
    """Allocate the KV pool and patch the model; returns the block count."""
    num_blocks = qwen3_cache_allocator(model, config, memory_utilization, block_size, dtype, device)
    qwen3_model_patcher(model, get_context)
    return num_blocks
