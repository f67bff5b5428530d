"""The committed golden fixtures (tests/golden/*.safetensors) still match the
oracle that wrote them (tests/golden/make_golden.py), on the CPU.

Elementwise results (norm/RoPE, the stores) must be identical; the attention
outputs, whose fp32 reductions may be ordered differently by another thread
count, must agree to one bf16 ulp.
"""

import importlib.util
from pathlib import Path

import pytest
import torch
from safetensors.torch import load_file

GOLDEN = Path(__file__).resolve().parent / "golden"
_spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
make_golden = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)


@pytest.mark.parametrize("name", sorted(make_golden.FIXTURES))
def test_fixture_reproduced_by_oracle(name):
    stored = load_file(str(GOLDEN / f"{name}.safetensors"))
    fresh = make_golden.FIXTURES[name]()
    assert set(stored) == set(fresh)
    for key, ref in stored.items():
        new = fresh[key].contiguous()
        assert new.dtype == ref.dtype and new.shape == ref.shape, key
        if key == "out":
            assert (new.float() - ref.float()).abs().max().item() <= 2 ** -7 * ref.float().abs().max().item(), key
        else:
            assert torch.equal(new, ref), key


def test_fixture_invariants():
    """Facts the fixtures must show whatever the oracle: a 1-token decode is
    the stored V row; the store leaves untouched slots alone."""
    d = load_file(str(GOLDEN / "paged_decode.safetensors"))
    page = int(d["block_tables"][0, 0])
    for h in range(8):
        assert torch.equal(d["out"][0, h], d["v_cache"][page, h // 4, 0])
    s = load_file(str(GOLDEN / "store.safetensors"))
    changed = (s["k_cache_out"] != s["k_cache"]).any(dim=-1)  # (NB, Hkv, BS)
    assert int(changed.sum()) <= 2 * (6 + 5)
