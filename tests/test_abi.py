"""The C ABI of libtsa.so, checked without a GPU (no compute calls).

* every entry point declared in include/tsa_api.h is exported by the library
  and bound by the Python shim;
* the ABI version matches;
* malformed arguments are rejected before anything touches a device, with
  TSA_ERR_INVALID and a message (NULL views, wrong ranks, dtype mismatches,
  GQA divisibility, mapping lengths), and unimplemented shapes with
  TSA_ERR_UNSUPPORTED;
* the decode workspace size follows the split plan.
"""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from tinyserver_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tsa_api.h"


def declared_symbols():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(tsa_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_are_exported_and_bound():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), f"{name} missing from libtsa.so"
        assert name in _lib.SIGNATURES, f"{name} not bound in tinyserver_amd._lib"
    assert set(_lib.SIGNATURES) == set(names)


def test_abi_version():
    assert _lib.load().tsa_abi_version() == _lib.ABI_VERSION


def _v(shape, dtype=torch.bfloat16, data=0x10000):
    """A view of a fake device address (never dereferenced: validation fails first)."""
    v = _lib.TsaView()
    v.data = data
    st = 1
    strides = []
    for n in reversed(shape):
        strides.append(st)
        st *= n
    for i, (n, s) in enumerate(zip(shape, reversed(strides))):
        v.size[i] = n
        v.stride[i] = s
    v.ndim = len(shape)
    v.dtype = _lib._DTYPES[dtype]
    return v


def _call(name, *args):
    lib = _lib.load()
    return getattr(lib, name)(*args), lib.tsa_last_error().decode()


R = ctypes.byref


def test_store_validation():
    rc, msg = _call("tsa_store_kv_mapped", None, None, None, None, None, None, None)
    assert rc == _lib.TSA_ERR_INVALID and "3D" in msg
    k2d = _v((2, 8))
    rc, msg = _call("tsa_store_kv_mapped", R(k2d), R(_v((2, 1, 8))), R(_v((1, 2, 4, 8))), R(_v((1, 2, 4, 8))),
                    R(_v((1,), torch.int32)), R(_v((1,), torch.int32)), None)
    assert rc == _lib.TSA_ERR_INVALID and "3D" in msg
    rc, msg = _call("tsa_store_kv_mapped", R(_v((2, 4, 8))), R(_v((2, 4, 8))), R(_v((2, 2, 4, 8))),
                    R(_v((2, 2, 4, 8))), R(_v((3,), torch.int32)), R(_v((4,), torch.int32)), None)
    assert rc == _lib.TSA_ERR_INVALID and "num_tokens" in msg
    rc, msg = _call("tsa_store_kv_mapped", R(_v((2, 4, 8))), R(_v((2, 4, 8), torch.float16)), R(_v((2, 2, 4, 8))),
                    R(_v((2, 2, 4, 8))), R(_v((4,), torch.int32)), R(_v((4,), torch.int32)), None)
    assert rc == _lib.TSA_ERR_INVALID and "dtype" in msg
    rc, msg = _call("tsa_store_kv_paged", R(_v((2, 4, 8))), R(_v((2, 4, 8))), R(_v((2, 2, 4, 8))),
                    R(_v((2, 2, 4, 8))), R(_v((2, 3), torch.int32)), R(_v((2,), torch.int32)), None, None)
    assert rc == _lib.TSA_ERR_INVALID and "cu_seqlens" in msg


def test_decode_validation():
    q = _v((4, 8, 128))
    kc = _v((10, 3, 16, 128))
    bt = _v((4, 2), torch.int32)
    sl = _v((4,), torch.int32)
    rc, msg = _call("tsa_paged_decode", R(q), R(q), R(kc), R(kc), R(bt), R(sl), 0.1, None, 0, 0, None)
    assert rc == _lib.TSA_ERR_INVALID and "multiple" in msg
    rc, msg = _call("tsa_paged_decode", R(_v((4, 128))), R(_v((4, 128))), R(kc), R(kc), R(bt), R(sl), 0.1, None, 0, 0,
                    None)
    assert rc == _lib.TSA_ERR_INVALID and "3D" in msg
    big = _v((4, 8, 1024))
    kcb = _v((10, 2, 16, 1024))
    rc, msg = _call("tsa_paged_decode", R(big), R(big), R(kcb), R(kcb), R(bt), R(sl), 0.1, None, 0, 0, None)
    assert rc == _lib.TSA_ERR_UNSUPPORTED
    # 60000 sequences x 2^20-token tables: more 16-token tiles than the
    # kernel's 32-bit tile prefix holds, rejected before any device work.
    n = 60000
    qn, btn, sln = _v((n, 8, 128)), _v((n, 1 << 16), torch.int32), _v((n,), torch.int32)
    kcn = _v((10, 2, 16, 128))
    rc, msg = _call("tsa_paged_decode", R(qn), R(qn), R(kcn), R(kcn), R(btn), R(sln), 0.1, None, 0, 0, None)
    assert rc == _lib.TSA_ERR_INVALID and "2^31" in msg


def test_noalloc_rejects_oversized_before_device_work():
    """tsa_paged_decode_noalloc refuses a call whose partials exceed the 16 MiB
    per-GPU scratch, from the shapes alone (no device is touched)."""
    q = _v((8192, 64, 128))
    kc = _v((4, 8, 16, 128))
    bt = _v((8192, 1), torch.int32)
    sl = _v((8192,), torch.int32)
    rc, msg = _call("tsa_paged_decode_noalloc", R(q), R(q), R(kc), R(kc), R(bt), R(sl), 0.1, 0, None)
    assert rc == _lib.TSA_ERR_INVALID and "bytes of scratch" in msg and "16777216" in msg
    need = _lib.load().tsa_paged_decode_workspace_bytes(8192, 64, 8, 128, 1, 16, 0)
    assert str(need) in msg


def test_noalloc_checks_arguments_first():
    """tsa_paged_decode_noalloc runs every argument check before it looks up
    its scratch (no device is touched): a malformed call gets the same
    message tsa_paged_decode gives."""
    q, kc = _v((4, 8, 128)), _v((10, 2, 16, 128))
    bt, sl = _v((4, 2), torch.int32), _v((4,), torch.int32)
    bad = _v((4, 7, 128))
    rc, msg = _call("tsa_paged_decode_noalloc", R(bad), R(bad), R(kc), R(kc), R(bt), R(sl), 0.1, 0, None)
    assert rc == _lib.TSA_ERR_INVALID and "multiple" in msg
    rc, msg = _call("tsa_paged_decode_noalloc", R(q), R(q), R(kc), R(kc), R(_v((3, 2), torch.int32)), R(sl), 0.1,
                    0, None)
    assert rc == _lib.TSA_ERR_INVALID and "num_seqs" in msg


def test_mixed_attention_shim_rank_checks():
    """The Python shim checks the cache and table ranks before it sizes the
    workspace: wrong ranks raise ValueError, as paged_attention_forward's do."""
    from tinyserver_amd.kernels import mixed_attention

    pq, pk = torch.zeros(10, 8, 128), torch.zeros(10, 2, 128)
    cu = torch.tensor([0, 4, 10], dtype=torch.int32)
    q, kc = torch.zeros(4, 8, 128), torch.zeros(10, 2, 16, 128)
    bt, sl = torch.zeros(4, 2, dtype=torch.int32), torch.ones(4, dtype=torch.int32)
    with pytest.raises(ValueError, match="4D"):
        mixed_attention(pq, pk, pk, cu, 6, q, kc[0], kc[0], bt, sl)
    with pytest.raises(ValueError, match="2D"):
        mixed_attention(pq, pk, pk, cu, 6, q, kc, kc, bt[0], sl)


def test_prefill_validation():
    q, k = _v((10, 6, 64)), _v((10, 4, 64))
    cu = _v((3,), torch.int32)
    rc, msg = _call("tsa_varlen_prefill", R(q), R(q), R(k), R(k), R(cu), R(cu), 5, 5, 1, 0.1, None)
    assert rc == _lib.TSA_ERR_INVALID and "divisible" in msg


def test_mixed_attention_validation():
    """tsa_mixed_attention checks both halves' arguments, as the two calls it
    replaces do, before any device work."""
    pq, pk = _v((10, 8, 128)), _v((10, 2, 128))
    cu = _v((3,), torch.int32)
    q = _v((4, 8, 128))
    kc = _v((10, 2, 16, 128))
    bt, sl = _v((4, 2), torch.int32), _v((4,), torch.int32)
    lib = _lib.load()
    ws_bytes = lib.tsa_paged_decode_workspace_bytes(4, 8, 2, 128, 2, 16, 0)
    ws = 1 << 20  # a fake, 256-byte aligned address: never dereferenced

    def call(p_k=pk, query=q, ws_ptr=ws, pwg=0):
        return _call("tsa_mixed_attention", R(pq), R(pq), R(p_k), R(p_k), R(cu), 9, 0.1, R(query), R(query), R(kc),
                     R(kc), R(bt), R(sl), 0.1, ws_ptr, ws_bytes, 0, pwg, None)

    rc, msg = call(p_k=_v((10, 3, 128)))
    assert rc == _lib.TSA_ERR_INVALID and "divisible" in msg
    rc, msg = call(query=_v((4, 7, 128)))
    assert rc == _lib.TSA_ERR_INVALID and "multiple" in msg
    rc, msg = call(ws_ptr=None)
    assert rc == _lib.TSA_ERR_INVALID and "workspace" in msg
    rc, msg = call(pwg=-1)
    assert rc == _lib.TSA_ERR_INVALID and "prefill_workgroups" in msg


def test_norm_rope_validation():
    q, k = _v((5, 4, 128)), _v((5, 2, 128))
    w, cs = _v((128,)), _v((5, 128))
    bad_w = _v((64,))
    rc, msg = _call("tsa_qk_norm_rope", R(q), R(k), R(q), R(k), R(bad_w), R(w), R(cs), R(cs), 1e-6, None)
    assert rc == _lib.TSA_ERR_INVALID and "head_dim" in msg
    rc, msg = _call("tsa_qk_norm_rope", R(q), R(k), R(q), R(k), R(w), R(w), R(_v((5, 128), torch.float32)), R(cs),
                    1e-6, None)
    assert rc == _lib.TSA_ERR_INVALID and "dtype" in msg


def test_workspace_plan():
    lib = _lib.load()
    # One partial slot of (acc[G][D], m[G], l[G]) per (unit, wave worker) pair
    # that can occur -- units + 4 * workgroups -- plus the tile prefix.
    n = lib.tsa_paged_decode_workspace_bytes(2, 8, 2, 128, 64, 16, 10)
    assert n >= (2 * 2 + 4 * 10) * 4 * (128 + 2) * 4 + 3 * 4
    assert lib.tsa_paged_decode_workspace_bytes(0, 8, 2, 128, 64, 16, 10) == 0


def test_workspace_plan_small_tables():
    """With no grid asked for: at most 64 (sequence, kv head) units whose
    tables hold at most 512 tokens run one workgroup per unit, whose partials
    stay in LDS, so the workspace is the tile prefix alone. Otherwise block
    tables of few tiles (Hkv * B * ceil(max_blocks * block_size / 16), at
    most 8 per default workgroup) take a grid of one workgroup per 8 such
    tiles, at least 64: the workspace holds units + 4 * workgroups partial
    slots."""
    lib = _lib.load()

    def plan(b, blocks, bs=16, nwg=0):
        return lib.tsa_paged_decode_workspace_bytes(b, 16, 8, 128, blocks, bs, nwg)

    def size(b, wg):  # G = 2, head_dim 128
        align = lambda n: (n + 255) // 256 * 256
        return align((b * 8 + 4 * wg) * 2 * (128 + 2) * 4) + align((b + 1) * 4)

    prefix_only = 256  # (B + 1) int32, 256-byte aligned
    assert plan(4, 32) == prefix_only  # the Qwen3-0.6B batch of 4 at contexts up to 512: 32 units
    assert plan(4, 16, bs=32) == prefix_only  # the same tokens in 32-token pages
    assert plan(8, 1) == prefix_only  # 64 units
    assert plan(4, 33) == size(4, 132)  # 528-token tables: the stream, 1056 tiles over 132 workgroups
    assert plan(9, 1) == size(9, 64)  # 72 units: the stream, the floor of 64 workgroups
    assert plan(4, 32, nwg=200) == size(4, 200)  # a grid asked for is kept
    assert plan(64, 256) > size(64, 128)  # the Qwen3-8B batch: the default grid (one per CU)


def test_sampling_workspace_plan():
    lib = _lib.load()
    # Split rows: 512 / B segments per row (2 .. 16), each a 32-byte
    # statistics record and 2048 buckets of a 4-byte count and an 8-byte mass.
    segs = 64 * 8
    assert lib.tsa_sample_tokens_workspace_bytes(64, 151936) >= segs * (32 + 2048 * 12)
    assert lib.tsa_sample_tokens_workspace_bytes(1, 151936) >= 16 * (32 + 2048 * 12)
    assert lib.tsa_sample_tokens_workspace_bytes(256, 151936) >= 256 * 2 * (32 + 2048 * 12)
    # No split: a batch that fills the device one row per workgroup, or short rows.
    assert lib.tsa_sample_tokens_workspace_bytes(257, 151936) == 0
    assert lib.tsa_sample_tokens_workspace_bytes(64, 4096) == 0
    assert lib.tsa_sample_tokens_workspace_bytes(0, 151936) == 0
