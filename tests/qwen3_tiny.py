"""A tiny random-init Qwen3 (local config, nothing downloaded) and helpers
that drive it the way the reference's tests do
(tests/model/paged_helpers.py:21-140): flattened prefill / decode inputs under
an InferenceContext for the patched model, and per-sequence full forwards of
the stock HF model as the baseline."""

from __future__ import annotations

import copy
import math

import torch
from transformers import Qwen3Config, Qwen3ForCausalLM

from tinyserver_amd.inference_context import InferenceContext, inference_context


def tiny_config(head_dim=128):
    return Qwen3Config(vocab_size=384, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=head_dim, rms_norm_eps=1e-6,
                       rope_theta=1e6, max_position_embeddings=2048, tie_word_embeddings=False,
                       attn_implementation="eager")


def tiny_models(dtype, device, block_size, num_blocks, seed=0):
    """(stock model, patched model with its own KV pool), same weights."""
    from tinyserver_amd.patches import qwen3_model_patcher

    torch.manual_seed(seed)
    cfg = tiny_config()
    base = Qwen3ForCausalLM(cfg).to(dtype=dtype, device=device).eval()
    patched = copy.deepcopy(base)
    pool = torch.zeros(2, cfg.num_hidden_layers, num_blocks, cfg.num_key_value_heads, block_size, cfg.head_dim,
                       dtype=dtype, device=device)
    for i, layer in enumerate(patched.model.layers):
        layer.self_attn.k_cache = pool[0, i]
        layer.self_attn.v_cache = pool[1, i]
    qwen3_model_patcher(patched)
    return base, patched


def allocate_block_tables(max_tokens, block_size):
    tables, nxt = [], 0
    for n in max_tokens:
        nb = max(1, math.ceil(n / block_size))
        tables.append(list(range(nxt, nxt + nb)))
        nxt += nb
    return tables


def patched_prefill_logits(model, prompts, tables, device):
    ids = [t for p in prompts for t in p]
    pos = [i for p in prompts for i in range(len(p))]
    ctx = InferenceContext(mode="prefill",
                           sequences=[{"num_tokens": len(p), "block_table": bt} for p, bt in zip(prompts, tables)])
    with torch.no_grad(), inference_context(ctx):
        out = model(input_ids=torch.tensor([ids], device=device), position_ids=torch.tensor([pos], device=device),
                    use_cache=False)
    last = torch.tensor(prompts_last_index(prompts), device=device)
    return out.logits[0, last]


def prompts_last_index(prompts):
    idx, off = [], 0
    for p in prompts:
        off += len(p)
        idx.append(off - 1)
    return idx


def patched_decode_logits(model, tokens, positions, tables, device):
    ctx = InferenceContext(mode="decode", sequences=[{"num_tokens": 1, "block_table": bt} for bt in tables])
    with torch.no_grad(), inference_context(ctx):
        out = model(input_ids=torch.tensor([tokens], device=device),
                    position_ids=torch.tensor([positions], device=device), use_cache=False)
    return out.logits[0]


def original_last_logits(model, ids, device):
    with torch.no_grad():
        out = model(input_ids=torch.tensor([ids], device=device), use_cache=False)
    return out.logits[0, -1]
