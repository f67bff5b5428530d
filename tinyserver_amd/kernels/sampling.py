"""Drop-in for tinyserver's batched sampler, ``sample_tokens``
(server/model/sampling.py:119-194), on the gfx950 HIP library.

Same signature, argument meaning and ValueError messages. One launch samples
every row (three for a small batch of long 16-bit rows, whose statistics and
histogram passes are spread over several workgroups per row, through a
workspace allocated here); nothing synchronises with the host (the caller's
``.tolist()`` is the step's one sync, as in the reference). The kernel finds the top-k cut, the
top-p cut and the inverse-CDF pick without sorting the row; its decisions
match the reference's sort/softmax/cumsum/searchsorted except where a target
lies within fp32 rounding of a cumulative sum.
"""

from __future__ import annotations

import torch

from .. import _lib


def _check_param(name: str, tensor: torch.Tensor, batch_size: int) -> None:
    # sampling.py:112-116
    if tensor.shape != (batch_size,):
        raise ValueError(f"Expected {name} shape [{batch_size}], got {tuple(tensor.shape)}")


def sample_tokens(
    logits: torch.Tensor,  # [B, V]
    temperature: torch.Tensor,  # [B]
    top_k: torch.Tensor,  # [B], 0 disables
    top_p: torch.Tensor,  # [B], 1.0 disables
    uniforms: torch.Tensor,  # [B] in [0, 1)
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One token per row: temperature scaling, top-k, then top-p over the
    survivors, then the first rank whose cumulative mass reaches
    ``uniforms * kept mass``; rows with temperature <= 0 take the argmax
    (lowest index on ties). Returns [B] int64 on the logits' device."""
    if logits.ndim != 2:
        raise ValueError(f"Expected logits shape [B, vocab_size], got {logits.ndim}D")
    batch_size, _ = logits.shape
    _check_param("temperature", temperature, batch_size)
    _check_param("top_k", top_k, batch_size)
    _check_param("top_p", top_p, batch_size)
    _check_param("uniforms", uniforms, batch_size)
    dev = _lib.require_device(logits, temperature, top_k, top_p, uniforms)
    if logits.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        logits = logits.float()
    temperature, top_p, uniforms = temperature.float(), top_p.float(), uniforms.float()
    if top_k.dtype not in (torch.int32, torch.int64):
        top_k = top_k.long()
    if out is None:
        out = torch.empty(batch_size, dtype=torch.int64, device=dev)
    lib = _lib.load()
    views = [_lib.view(t) for t in (out, logits, temperature, top_k, top_p, uniforms)]
    nbytes = _workspace_bytes(lib, *logits.shape)
    if nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        rc = lib.tsa_sample_tokens_ws(*map(_lib.ref, views), ws.data_ptr(), nbytes, _lib.stream_of(dev))
    else:
        rc = lib.tsa_sample_tokens(*map(_lib.ref, views), _lib.stream_of(dev))
    _lib.check(rc, "sample_tokens")
    return out


_WS_BYTES: dict = {}


def _workspace_bytes(lib, batch: int, vocab: int) -> int:
    key = (batch, vocab)
    if key not in _WS_BYTES:
        _WS_BYTES[key] = int(lib.tsa_sample_tokens_workspace_bytes(batch, vocab))
    return _WS_BYTES[key]
