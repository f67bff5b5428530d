"""The patched Qwen3 forward on the gfx950 kernels against stock HF.

Ports the reference's model-level check (tests/model/test_paged_attention_
validation.py:27-30, 38-110): last-token logits of a multi-sequence prefill,
then several batched decode steps, each compared with a full forward of the
unpatched model over the same tokens -- in fp32 with the reference's
tolerances (prefill 1e-4, decode 1e-3, page 4). The model is a tiny random-init
Qwen3 (local config; the reference's tests download Qwen3-0.6B). In bf16 (page
16, the production setting) whole-model logits carry each implementation's own
bf16 rounding, so the patched model is held to the stock model's accuracy: both
are compared with an fp32 forward of the same (bf16-valued) weights, and the
patched model's error may not exceed the stock bf16 model's by more than a
small margin.
"""

import copy

import pytest
import torch

from tests.helpers import assert_close
from tests.qwen3_tiny import (allocate_block_tables, original_last_logits, patched_decode_logits,
                              patched_prefill_logits, tiny_models)

pytestmark = pytest.mark.gpu
DEV = "cuda"

PROMPTS = [[(7 * i + 3) % 384 for i in range(n)] for n in (5, 17, 33)]


def _run(dtype, block_size, prefill_tol, decode_tol, steps=4):
    tables = allocate_block_tables([len(p) + steps + 1 for p in PROMPTS], block_size)
    base, patched = tiny_models(dtype, DEV, block_size, sum(len(t) for t in tables) + 2)
    logits = patched_prefill_logits(patched, PROMPTS, tables, DEV)
    seqs = [list(p) for p in PROMPTS]
    for i, p in enumerate(seqs):
        ref = original_last_logits(base, p, DEV)
        assert_close(logits[i], ref, what=f"{dtype} prefill seq {i}", **prefill_tol)
    for step in range(steps):
        nxt = [int(logits[i].argmax()) for i in range(len(seqs))]
        positions = [len(s) for s in seqs]
        for s, t in zip(seqs, nxt):
            s.append(t)
        logits = patched_decode_logits(patched, nxt, positions, tables, DEV)
        for i, s in enumerate(seqs):
            ref = original_last_logits(base, s, DEV)
            assert_close(logits[i], ref, what=f"{dtype} decode step {step} seq {i}", **decode_tol)


def test_fp32_matches_stock_model():
    _run(torch.float32, 4, dict(max_abs=1e-4, mean_abs=1e-5), dict(max_abs=1e-3, mean_abs=1e-4))


def _err(a, b):
    d = (a.float() - b.float()).abs()
    return d.max().item(), d.mean().item()


def test_bf16_as_accurate_as_stock_model(steps=4):
    block_size = 16
    tables = allocate_block_tables([len(p) + steps + 1 for p in PROMPTS], block_size)
    base, patched = tiny_models(torch.bfloat16, DEV, block_size, sum(len(t) for t in tables) + 2)
    exact = copy.deepcopy(base).float()  # same bf16-valued weights, fp32 arithmetic
    logits = patched_prefill_logits(patched, PROMPTS, tables, DEV)
    seqs = [list(p) for p in PROMPTS]
    for step in range(steps + 1):
        for i, s in enumerate(seqs):
            ref = original_last_logits(exact, s, DEV)
            mine = _err(logits[i], ref)
            stock = _err(original_last_logits(base, s, DEV), ref)
            print(f"step {step} seq {i}: patched vs fp32 max {mine[0]:.3e} mean {mine[1]:.3e}; "
                  f"stock bf16 vs fp32 max {stock[0]:.3e} mean {stock[1]:.3e}", flush=True)
            assert mine[1] <= 1.5 * stock[1] + 1e-4, f"step {step} seq {i}: mean error {mine[1]:.3e} vs stock {stock[1]:.3e}"
            assert mine[0] <= 2.0 * stock[0] + 1e-3, f"step {step} seq {i}: max error {mine[0]:.3e} vs stock {stock[0]:.3e}"
        if step == steps:
            break
        nxt = [int(logits[i].argmax()) for i in range(len(seqs))]
        positions = [len(s) for s in seqs]
        for s, t in zip(seqs, nxt):
            s.append(t)
        logits = patched_decode_logits(patched, nxt, positions, tables, DEV)


def test_fused_decode_route_matches_two_launches(monkeypatch):
    """Small decode steps take the single-launch fused step; larger ones the
    norm/store launch followed by paged attention. Both routes give the same
    logits, bit for bit, and leave the same caches."""
    from tinyserver_amd.patches import qwen3 as glue

    block_size, steps = 16, 3
    tables = allocate_block_tables([len(p) + steps + 1 for p in PROMPTS], block_size)
    runs = []
    for max_tiles in (glue.FUSED_DECODE_MAX_TILES, -1):  # -1: every step takes the two-launch route
        monkeypatch.setattr(glue, "FUSED_DECODE_MAX_TILES", max_tiles)
        _, patched = tiny_models(torch.bfloat16, DEV, block_size, sum(len(t) for t in tables) + 2)
        logits = patched_prefill_logits(patched, PROMPTS, tables, DEV)
        seqs = [list(p) for p in PROMPTS]
        out = []
        for _ in range(steps):
            nxt = [int(logits[i].argmax()) for i in range(len(seqs))]
            positions = [len(s) for s in seqs]
            for s, t in zip(seqs, nxt):
                s.append(t)
            logits = patched_decode_logits(patched, nxt, positions, tables, DEV)
            out.append(logits.clone())
        layer = patched.model.layers[0].self_attn
        runs.append((out, layer.k_cache.clone(), layer.v_cache.clone()))
    (a, ka, va), (b, kb, vb) = runs
    for step, (x, y) in enumerate(zip(a, b)):
        assert torch.equal(x, y), f"decode step {step}: fused and two-launch logits differ"
    assert torch.equal(ka, kb) and torch.equal(va, vb)
