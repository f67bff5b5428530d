"""Host logic of the Qwen3 call-site glue, on the CPU (no kernel launches).

* the device metadata matches the reference's per-layer construction
  (server/model/patches/qwen3.py:296-310, 388-400): zero-padded int32 block
  tables, cu_seqlens over num_tokens, seq_lens = position + 1; tables and
  cu_seqlens share one packed buffer (one transfer);
* the reference's ValueErrors (:182-187, :329-330);
* one build per forward: layers that get the same position_ids reuse it, a
  new step's tensor rebuilds it;
* the glue takes the reference engine's own context: a plain
  ``InferenceContext{mode, sequences}`` dataclass
  (server/model/inference_context.py:18-21, decode entries holding only
  "block_table" as engine.py:579-582 builds them), read through the engine
  module's getter when that module imports;
* the patched forward has no CPU path;
* the device-resident block tables (BlockTableMirror) equal the padded
  tables the reference builds, step after step, while uploading only the
  blocks appended since a list was last seen (the BlockManager's lists only
  grow in place, server/model/block_manager.py:102-159).
"""

import sys
import types
from dataclasses import dataclass, field
from typing import Any

import pytest
import torch

from tinyserver_amd.inference_context import InferenceContext, get_inference_context, inference_context
from tinyserver_amd.patches import device_metadata
from tinyserver_amd.patches import qwen3 as patch_mod
from tinyserver_amd.patches.block_tables import BlockTableMirror

CPU = torch.device("cpu")


def test_prefill_metadata():
    ctx = InferenceContext("prefill", [{"num_tokens": 3, "block_table": [4, 9]}, {"num_tokens": 1, "block_table": [2]},
                                       {"num_tokens": 5, "block_table": [0, 1, 7]}])
    pos = torch.tensor([[0, 1, 2, 0, 0, 1, 2, 3, 4]])
    m = device_metadata(ctx, pos, 9, CPU)
    assert m.block_tables.dtype == torch.int32 and m.block_tables.tolist() == [[4, 9, 0], [2, 0, 0], [0, 1, 7]]
    assert m.cu_seqlens.tolist() == [0, 3, 4, 9] and m.max_seqlen == 5
    assert m.positions is None and m.seq_lens is None


def test_decode_metadata():
    ctx = InferenceContext("decode", [{"num_tokens": 1, "block_table": [3]}, {"num_tokens": 1, "block_table": [5, 6]}])
    m = device_metadata(ctx, torch.tensor([[15, 16]]), 2, CPU)
    assert m.block_tables.tolist() == [[3, 0], [5, 6]]
    assert m.cu_seqlens.tolist() == [0, 1, 2]
    assert m.positions.tolist() == [15, 16] and m.seq_lens.tolist() == [16, 17]
    assert m.seq_lens.dtype == torch.int32
    assert m.table_slots == 3  # the KV size the glue uses to choose the fused decode step


def test_reference_errors():
    ctx = InferenceContext("prefill", [{"num_tokens": 3, "block_table": [0]}])
    with pytest.raises(ValueError, match="sum to 3"):
        device_metadata(ctx, torch.zeros(1, 4, dtype=torch.long), 4, CPU)
    ctx = InferenceContext("prefill", [{"num_tokens": 0, "block_table": [0]}, {"num_tokens": 2, "block_table": [1]}])
    with pytest.raises(ValueError, match="positive"):
        device_metadata(ctx, torch.zeros(1, 2, dtype=torch.long), 2, CPU)
    ctx = InferenceContext("decode", [{"num_tokens": 1, "block_table": [0]}])
    with pytest.raises(ValueError, match="Position ids"):
        device_metadata(ctx, None, 1, CPU)


def test_one_build_per_forward():
    ctx = InferenceContext("decode", [{"num_tokens": 1, "block_table": [3]}])
    pos = torch.tensor([[7]])
    a = device_metadata(ctx, pos, 1, CPU)
    assert device_metadata(ctx, pos, 1, CPU) is a  # the next layer of the same forward
    b = device_metadata(ctx, torch.tensor([[8]]), 1, CPU)  # the next step
    assert b is not a and b.positions.tolist() == [8]
    pos2 = torch.tensor([[9]])
    c = device_metadata(ctx, pos2, 1, CPU)
    pos2.add_(1)  # changed in place: rebuilt
    assert device_metadata(ctx, pos2, 1, CPU).positions.tolist() == [10] and c.positions.tolist() == [9]


def test_context_swap():
    outer = get_inference_context()
    ctx = InferenceContext("decode", [])
    with inference_context(ctx):
        assert get_inference_context() is ctx
    assert get_inference_context() is outer


def test_patched_forward_has_no_cpu_path():
    from tests.qwen3_tiny import tiny_models

    _, patched = tiny_models(torch.float32, "cpu", 4, 8)
    ctx = InferenceContext("prefill", [{"num_tokens": 3, "block_table": [0]}])
    with torch.no_grad(), inference_context(ctx), pytest.raises(RuntimeError, match="GPU"):
        patched(input_ids=torch.tensor([[1, 2, 3]]), position_ids=torch.tensor([[0, 1, 2]]), use_cache=False)


@dataclass
class EngineContext:
    """The reference engine's context, field for field: nothing else on it."""

    mode: str = "prefill"
    sequences: list[dict[str, Any]] = field(default_factory=list)


def test_reference_shaped_context():
    assert set(EngineContext.__dataclass_fields__) == {"mode", "sequences"}
    ctx = EngineContext("decode", [{"block_table": [3]}, {"block_table": [5, 6]}])  # engine.py:579-582
    pos = torch.tensor([[15, 16]])
    m = device_metadata(ctx, pos, 2, CPU)
    assert m.block_tables.tolist() == [[3, 0], [5, 6]] and m.seq_lens.tolist() == [16, 17]
    assert device_metadata(ctx, pos, 2, CPU) is m  # the next layer reuses the build
    assert not hasattr(ctx, "_device_meta") and vars(ctx).keys() == {"mode", "sequences"}  # nothing stored on it
    # the next step: a new context object, even with the same position_ids tensor
    ctx2 = EngineContext("decode", [{"block_table": [4]}, {"block_table": [7, 8]}])
    m2 = device_metadata(ctx2, pos, 2, CPU)
    assert m2 is not m and m2.block_tables.tolist() == [[4, 0], [7, 8]]
    pre = EngineContext("prefill", [{"num_tokens": 2, "block_table": [1]}, {"num_tokens": 1, "block_table": [2]}])
    mp = device_metadata(pre, torch.tensor([[0, 1, 0]]), 3, CPU)
    assert mp.cu_seqlens.tolist() == [0, 2, 3] and mp.max_seqlen == 2


def test_context_without_weakref_support_is_rebuilt():
    class Slotted:
        __slots__ = ("mode", "sequences")

        def __init__(self, mode, sequences):
            self.mode, self.sequences = mode, sequences

    ctx = Slotted("decode", [{"block_table": [3]}])
    pos = torch.tensor([[7]])
    a = device_metadata(ctx, pos, 1, CPU)
    b = device_metadata(ctx, pos, 1, CPU)
    assert a is not b and a.positions.tolist() == b.positions.tolist() == [7]


@pytest.fixture
def engine_module(monkeypatch):
    """A module importable as server.model.inference_context with the
    reference's getter/context-manager contract (this package's stand-in for
    the engine; the reference itself is never imported)."""
    mod = types.ModuleType("server.model.inference_context")
    mod.InferenceContext = EngineContext
    mod.current = EngineContext()
    mod.get_inference_context = lambda: mod.current
    pkg, sub = types.ModuleType("server"), types.ModuleType("server.model")
    pkg.__path__, sub.__path__ = [], []
    pkg.model, sub.inference_context = sub, mod
    for name, m in (("server", pkg), ("server.model", sub), ("server.model.inference_context", mod)):
        monkeypatch.setitem(sys.modules, name, m)
    return mod


def test_getter_is_the_engines_when_importable(engine_module):
    assert patch_mod.engine_context_getter() is engine_module.get_inference_context


def test_getter_falls_back_to_the_mirror(monkeypatch):
    monkeypatch.setattr(patch_mod, "ENGINE_CONTEXT_MODULE", "no_such_engine_module.inference_context")
    assert patch_mod.engine_context_getter() is get_inference_context


def test_patched_forward_reads_the_engine_context(engine_module):
    from tests.qwen3_tiny import tiny_models

    _, patched = tiny_models(torch.float32, "cpu", 4, 8)
    # The engine's context says 2 prefill tokens for a 3-token input: the
    # reference's ValueError names the engine context's sum (this package's
    # own current context, empty, would say 0).
    engine_module.current = EngineContext("prefill", [{"num_tokens": 2, "block_table": [0]}])
    with torch.no_grad(), pytest.raises(ValueError, match="sum to 2"):
        patched(input_ids=torch.tensor([[1, 2, 3]]), position_ids=torch.tensor([[0, 1, 2]]), use_cache=False)


def _padded(tables):
    width = max(max((len(t) for t in tables), default=0), 1)
    return [list(t) + [0] * (width - len(t)) for t in tables]


def test_block_table_mirror_follows_the_lists():
    """A run of steps as the BlockManager drives its lists (allocate a fresh
    list, append one block every few steps, free = a new empty list, batches
    changing composition), on a mirror small enough to evict and grow: every
    gathered table equals the zero-padded tables, and a decode step uploads
    only the blocks appended since the step before."""
    g = torch.Generator().manual_seed(5)
    mirror = BlockTableMirror(CPU, rows=4, width=2)
    live = {}  # sequence -> its block list
    next_block = 0

    def new_list(n):
        nonlocal next_block
        blocks = list(range(next_block, next_block + n))
        next_block += n
        return blocks

    for step in range(200):
        r = torch.rand(3, generator=g).tolist()
        if r[0] < 0.15 or not live:  # a new sequence: allocate
            live[step] = new_list(int(1 + 6 * r[1]))
        if r[2] < 0.1 and len(live) > 1:  # a sequence finishes: free replaces its list
            seq = sorted(live)[int(r[1] * len(live))]
            live[seq] = []
            del live[seq]
        for seq, blocks in live.items():  # decode growth: one block now and then
            if (seq + step) % 7 == 0:
                blocks.append(next_block)
                next_block += 1
        batch = [live[s] for s in sorted(live) if (s + step) % 5 != 0] or [next(iter(live.values()))]
        before = mirror.uploaded
        appended = sum(len(b) - mirror.entries[id(b)].synced for b in batch
                       if id(b) in mirror.entries and mirror.entries[id(b)].blocks is b)
        new = sum(len(b) for b in batch if id(b) not in mirror.entries or mirror.entries[id(b)].blocks is not b)
        tables, extra = mirror.gather(batch, [len(batch)])
        assert tables.dtype == torch.int32 and tables.tolist() == _padded(batch), step
        assert extra.tolist() == [len(batch)]
        assert mirror.uploaded - before == appended + new  # appended tails and unseen lists only
    assert mirror.table.shape[0] > 4 or len(mirror.entries) <= 4


def test_block_table_mirror_rewrites_a_changed_list():
    mirror = BlockTableMirror(CPU, rows=2, width=4)
    a, b = [5, 6, 7], [8]
    assert mirror.gather([a, b])[0].tolist() == [[5, 6, 7], [8, 0, 0]]
    a[-1] = 9  # the last synced entry changed in place
    b.clear()  # shrank
    assert mirror.gather([a, b])[0].tolist() == [[5, 6, 9], [0, 0, 0]]
    c = [1, 2]  # a third list takes an evicted row: no stale entries past its end
    assert mirror.gather([c])[0].tolist() == [[1, 2]]
    assert mirror.gather([c, a])[0].tolist() == [[1, 2, 0], [5, 6, 9]]


def test_decode_steps_upload_appended_blocks_only():
    """Through device_metadata: after the first step, steps upload only the
    blocks the sequences gained."""
    lists = [[3, 4], [5]]
    ctx = InferenceContext("decode", [{"block_table": t} for t in lists])
    m = device_metadata(ctx, torch.tensor([[20, 3]]), 2, CPU)
    mirror = patch_mod._mirrors[CPU]
    assert m.block_tables.tolist() == [[3, 4], [5, 0]]
    before = mirror.uploaded
    lists[1].append(6)
    ctx = InferenceContext("decode", [{"block_table": t} for t in lists])
    m = device_metadata(ctx, torch.tensor([[21, 4]]), 2, CPU)
    assert m.block_tables.tolist() == [[3, 4], [5, 6]] and m.cu_seqlens.tolist() == [0, 1, 2]
    assert mirror.uploaded - before == 1
