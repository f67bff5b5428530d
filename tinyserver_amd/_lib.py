"""ctypes binding of libtsa.so (include/tsa_api.h).

Tensors cross the boundary as ``tsa_view`` structs (data pointer, sizes,
element strides, dtype); the HIP stream is torch's current stream on the
tensor's device. There is no CPU fallback: a missing library raises.
"""

from __future__ import annotations

import ctypes
import struct
from ctypes import c_double, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libtsa.so"

TSA_OK, TSA_ERR_INVALID, TSA_ERR_UNSUPPORTED, TSA_ERR_LAUNCH = 0, -1, -2, -3
TSA_BF16, TSA_F16, TSA_F32, TSA_I32, TSA_I64 = 0, 1, 2, 3, 4
_DTYPES = {
    torch.bfloat16: TSA_BF16,
    torch.float16: TSA_F16,
    torch.float32: TSA_F32,
    torch.int32: TSA_I32,
    torch.int64: TSA_I64,
}


class TsaView(ctypes.Structure):
    _fields_ = [
        ("data", c_void_p),
        ("size", c_int64 * 4),
        ("stride", c_int64 * 4),
        ("ndim", c_int32),
        ("dtype", c_int32),
    ]


# A view argument: the address of a tsa_view. view() hands over the packed
# bytes themselves (ctypes passes a bytes object's buffer as the pointer,
# valid for the call); a TsaView passed by ctypes.byref works too.
_V = c_void_p

# name -> (restype, argtypes); mirrors include/tsa_api.h.
SIGNATURES = {
    "tsa_abi_version": (c_int, []),
    "tsa_last_error": (ctypes.c_char_p, []),
    "tsa_store_kv": (c_int, [_V, _V, _V, _V, _V, c_int64, c_void_p]),
    "tsa_store_kv_mapped": (c_int, [_V, _V, _V, _V, _V, _V, c_void_p]),
    "tsa_store_kv_paged": (c_int, [_V, _V, _V, _V, _V, _V, _V, c_void_p]),
    "tsa_qk_norm_rope": (c_int, [_V, _V, _V, _V, _V, _V, _V, _V, c_double, c_void_p]),
    "tsa_qk_norm_rope_store": (
        c_int,
        [_V, _V, _V, _V, _V, _V, _V, _V, _V, c_double, _V, _V, _V, _V, _V, c_void_p],
    ),
    "tsa_paged_decode_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int32]),
    "tsa_paged_decode": (
        c_int,
        [_V, _V, _V, _V, _V, _V, c_double, c_void_p, c_size_t, c_int32, c_void_p],
    ),
    "tsa_paged_decode_noalloc": (c_int, [_V, _V, _V, _V, _V, _V, c_double, c_int32, c_void_p]),
    "tsa_paged_decode_step": (
        c_int,
        [_V] * 8 + [c_double] + [_V] * 4 + [c_double, c_void_p, c_size_t, c_int32, c_void_p],
    ),
    "tsa_varlen_prefill": (c_int, [_V, _V, _V, _V, _V, _V, c_int64, c_int64, c_int32, c_double, c_void_p]),
    "tsa_mixed_attention": (
        c_int,
        [_V] * 5 + [c_int64, c_double] + [_V] * 6 + [c_double, c_void_p, c_size_t, c_int32, c_int32, c_void_p],
    ),
    "tsa_sample_tokens": (c_int, [_V, _V, _V, _V, _V, _V, c_void_p]),
    "tsa_sample_tokens_workspace_bytes": (c_size_t, [c_int64, c_int64]),
    "tsa_sample_tokens_ws": (c_int, [_V, _V, _V, _V, _V, _V, c_void_p, c_size_t, c_void_p]),
}

ABI_VERSION = 1
_lib = None


def load() -> ctypes.CDLL:
    """Load libtsa.so once. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP library first "
                "(python -m tinyserver_amd._build or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.tsa_abi_version() != ABI_VERSION:
            raise RuntimeError(f"libtsa.so ABI {lib.tsa_abi_version()} != expected {ABI_VERSION}")
        _lib = lib
    return _lib


# One struct.pack per view (the layout of tsa_view; unused entries stay zero)
# instead of ctypes field sets, which cost microseconds per call.
_PACK = [struct.Struct("<Q" + "q" * nd + "x" * (8 * (4 - nd)) + "q" * nd + "x" * (8 * (4 - nd)) + "ii")
         for nd in range(5)]


def view(t: torch.Tensor | None) -> bytes | None:
    """Describe a tensor for the C ABI: the tsa_view struct's bytes (None
    stays None -> NULL)."""
    if t is None:
        return None
    nd = t.dim()
    if nd > 4:
        raise ValueError(f"tensors of rank > 4 are not supported (got {nd})")
    dt = _DTYPES.get(t.dtype)
    if dt is None:
        raise ValueError(f"unsupported dtype {t.dtype}")
    return _PACK[nd].pack(t.data_ptr() if t.numel() else 0, *t.shape, *t.stride(), nd, dt)


def ref(v: bytes | None):
    """The argument for a view (its bytes; ctypes passes their address)."""
    return v


def check(rc: int, what: str) -> None:
    if rc == TSA_OK:
        return
    msg = (load().tsa_last_error() or b"").decode(errors="replace")
    if rc == TSA_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    if rc == TSA_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (status {rc})")


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one GPU; the kernels have no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("tinyserver_amd kernels run on a ROCm GPU; got a CPU tensor")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def stream_of(device: torch.device) -> int:
    """The raw handle of the device's current stream (no Stream object made)."""
    return torch._C._cuda_getCurrentRawStream(device.index if device.index is not None else torch.cuda.current_device())
