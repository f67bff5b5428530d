"""Per-step inference context read by the patched attention forward.

Mirrors server/model/inference_context.py:18-48: ``InferenceContext{mode,
sequences}`` with ``sequences[i] = {"num_tokens": int, "block_table":
list[int]}`` in the order of the flattened batch, a module-global current
context, and ``inference_context(ctx)`` to swap it for the duration of a
forward. As in the reference the global is unsynchronised: one engine thread
drives the forward and the swap.

The model patch reads the engine's own context module when it imports
(server.model.inference_context); this mirror serves when it does not. The
patch stores nothing on a context.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import Any, Iterator


@dataclass
class InferenceContext:
    mode: str = "prefill"
    sequences: list[dict[str, Any]] = field(default_factory=list)


_current = InferenceContext()


def get_inference_context() -> InferenceContext:
    """The context of the forward in progress."""
    return _current


@contextmanager
def inference_context(ctx: InferenceContext) -> Iterator[InferenceContext]:
    """Make ``ctx`` current inside the block; restore the previous one after."""
    global _current
    previous, _current = _current, ctx
    try:
        yield ctx
    finally:
        _current = previous
