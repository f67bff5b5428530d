"""Host logic of the Qwen3 call-site glue, on the CPU (no kernel launches).

* the device metadata matches the reference's per-layer construction
  (server/model/patches/qwen3.py:296-310, 388-400): zero-padded int32 block
  tables, cu_seqlens over num_tokens, seq_lens = position + 1; tables and
  cu_seqlens share one packed buffer (one transfer);
* the reference's ValueErrors (:182-187, :329-330);
* one build per forward: layers that get the same position_ids reuse it, a
  new step's tensor rebuilds it;
* the patched forward has no CPU path.
"""

import pytest
import torch

from tinyserver_amd.inference_context import InferenceContext, get_inference_context, inference_context
from tinyserver_amd.patches import device_metadata

CPU = torch.device("cpu")


def test_prefill_metadata():
    ctx = InferenceContext("prefill", [{"num_tokens": 3, "block_table": [4, 9]}, {"num_tokens": 1, "block_table": [2]},
                                       {"num_tokens": 5, "block_table": [0, 1, 7]}])
    pos = torch.tensor([[0, 1, 2, 0, 0, 1, 2, 3, 4]])
    m = device_metadata(ctx, pos, 9, CPU)
    assert m.block_tables.dtype == torch.int32 and m.block_tables.tolist() == [[4, 9, 0], [2, 0, 0], [0, 1, 7]]
    assert m.cu_seqlens.tolist() == [0, 3, 4, 9] and m.max_seqlen == 5
    assert m.positions is None and m.seq_lens is None
    # one packed buffer, so one host-to-device transfer
    assert m.block_tables.untyped_storage().data_ptr() == m.cu_seqlens.untyped_storage().data_ptr()


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
