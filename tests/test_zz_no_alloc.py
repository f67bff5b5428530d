"""tsa_paged_decode_noalloc (the decode entry point that allocates nothing)
through the C ABI, against tsa_paged_decode with a caller workspace: the
same kernels on the same inputs give bit-identical outputs. Two calls in a
row, the second with a smaller batch (the scratch keeps the first call's
contents, which the second must not see), then the first shape again; calls
the generic kernel serves (fp32, head_dim 96), which take no scratch; plus a
call that needs more scratch than the library holds, rejected before any
device work.
"""

import ctypes

import pytest
import torch

from tests.helpers import assert_bitexact
from tinyserver_amd import _lib
from tinyserver_amd import workloads as W
from tinyserver_amd.kernels import paged_attention_forward

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _noalloc(q, kc, vc, bt, sl, num_workgroups=0):
    lib = _lib.load()
    out = torch.empty_like(q)
    views = [_lib.view(t) for t in (out, q, kc, vc, bt, sl)]
    rc = lib.tsa_paged_decode_noalloc(*map(_lib.ref, views), q.shape[-1] ** -0.5, num_workgroups,
                                      torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "tsa_paged_decode_noalloc")
    return out


def _case(name, **kw):
    w = W.make(name, device=DEV, poison=True, **kw)
    return w.q, w.k_cache, w.v_cache, w.block_tables, w.ctx_lens.to(torch.int32).to(DEV)


def test_noalloc_matches_workspace_entry_point():
    big = _case("qwen3-8b-decode-bs64")
    small = _case("qwen3-0.6b-decode-bs4")
    for args in (big, small, big):
        got = _noalloc(*args)
        ref = paged_attention_forward(*args[:4], 16, args[4])
        torch.cuda.synchronize()
        assert_bitexact(got, ref, f"noalloc vs workspace, batch {args[0].shape[0]}")


def test_noalloc_grids_and_shapes():
    """Other worker grids and a 32-head GQA-8 batch, alternating, each equal
    to the workspace entry point's output."""
    a = _case("qwen3-32b-decode-bs32", ctx_lo=100, ctx_hi=3000, pool_slack=1.1)
    b = _case("qwen3-0.6b-decode-bs4")
    for args, nwg in ((a, 0), (b, 7), (a, 64), (b, 0)):
        got = _noalloc(*args, num_workgroups=nwg)
        ref = paged_attention_forward(*args[:4], 16, args[4], num_workgroups=nwg)
        torch.cuda.synchronize()
        assert_bitexact(got, ref, f"noalloc grid {nwg}")


def test_noalloc_rejects_oversized_calls():
    """A batch whose partials exceed the 16 MiB scratch is refused with a
    clear error, and nothing is launched."""
    q = torch.zeros(8192, 64, 128, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(4, 8, 16, 128, dtype=torch.bfloat16, device=DEV)
    bt = torch.zeros(8192, 1, dtype=torch.int32, device=DEV)
    sl = torch.ones(8192, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="bytes of scratch"):
        _noalloc(q, kc, kc, bt, sl)


def test_noalloc_generic_kernel_calls():
    """Calls the generic kernel serves need no scratch: fp32 and head_dim 96
    are accepted and equal the workspace entry point, bit for bit."""
    f32 = tuple(t.float() if t.is_floating_point() else t for t in _case("qwen3-0.6b-decode-bs4"))
    g = torch.Generator(device="cpu").manual_seed(5)
    q96 = torch.randn(3, 8, 96, generator=g).to(torch.bfloat16).to(DEV)
    kc96 = torch.randn(12, 2, 16, 96, generator=g).to(torch.bfloat16).to(DEV)
    vc96 = torch.randn(12, 2, 16, 96, generator=g).to(torch.bfloat16).to(DEV)
    bt96 = torch.randperm(12, generator=g)[:12].reshape(3, 4).to(torch.int32).to(DEV)
    sl96 = torch.tensor([1, 40, 64], dtype=torch.int32, device=DEV)
    for args in (f32, (q96, kc96, vc96, bt96, sl96), f32):
        got = _noalloc(*args)
        ref = paged_attention_forward(*args[:4], 16, args[4])
        torch.cuda.synchronize()
        assert_bitexact(got, ref, f"noalloc generic kernel, {args[0].dtype}, head_dim {args[0].shape[-1]}")
