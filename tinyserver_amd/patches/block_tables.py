"""A device-resident mirror of the engine's per-sequence block tables.

The reference's BlockManager gives each sequence one Python list of block ids
and only ever grows it in place: ``allocate`` assigns a fresh list
(server/model/block_manager.py:102-108), ``append_slot`` appends a block
(:134), ``free`` replaces it by a new empty list (:159). Every step's
InferenceContext carries those same list objects (engine.py:579-582 for a
decode step). The reference rebuilds a padded int32 table from the lists in
every layer (server/model/patches/qwen3.py:388-397) and copies it over.

The mirror keeps one device row per list it has seen and, per step, uploads
only what changed: the blocks appended since the last step (a decode step
adds at most one per sequence every block_size tokens) and whole rows for
lists it has not seen. The batch's (B, width) table is then gathered from
the mirror on the device in batch order. Per step that is one small
host-to-device transfer (the batch's row numbers, any extra int32 payload
such as cu_seqlens, and the changed entries), one scatter when entries
changed, and one gather, instead of the full padded table.

A list is tracked by identity while its entry holds a reference to it (so its
id cannot be reused), and checked for change by its length and its last
synced entry: a list that shrank or whose last synced entry differs is
uploaded whole again. Changing an entry other than the last one in place,
which the BlockManager never does, is not detected. Entries not in the
current batch are evicted least recently used first when rows run out; the
mirror grows when a batch needs more rows or a longer table than it has.

One stream per mirror: the scatter of a step's changed entries and the
gather of its table run on whatever stream is current, and nothing orders
them against another stream's use of the mirror. The reference engine runs
every forward on one stream, and the glue keeps one mirror per device; a
caller that drives steps from several streams needs one mirror per stream.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np
import torch


class _Entry:
    __slots__ = ("blocks", "row", "synced", "last", "seen")

    def __init__(self, blocks: list, row: int):
        self.blocks = blocks  # the engine's list (a reference keeps its id unique)
        self.row = row
        self.synced = 0       # entries of `blocks` already on the device
        self.last = None      # blocks[synced - 1] when it was uploaded
        self.seen = 0         # the last step it was in


class BlockTableMirror:
    """Device copy of the block tables of the sequences a device has seen."""

    def __init__(self, device: torch.device, rows: int = 256, width: int = 64):
        self.device = torch.device(device)
        self.table = torch.zeros(rows, width, dtype=torch.int32, device=self.device)
        self.row_len = [0] * rows        # nonzero prefix length of each device row
        self.free_rows = list(range(rows - 1, -1, -1))
        self.entries: dict[int, _Entry] = {}
        self.step = 0
        self.uploaded = 0                # block entries sent to the device so far (for tests and stats)

    def _grow(self, rows: int, width: int) -> None:
        old_rows, old_width = self.table.shape
        rows, width = max(rows, old_rows), max(width, old_width)
        if (rows, width) == (old_rows, old_width):
            return
        table = torch.zeros(rows, width, dtype=torch.int32, device=self.device)
        table[:old_rows, :old_width] = self.table
        self.table = table
        self.row_len += [0] * (rows - old_rows)
        self.free_rows = list(range(rows - 1, old_rows - 1, -1)) + self.free_rows

    def _take_row(self, batch: set, batch_size: int) -> int:
        if not self.free_rows:
            # Evict the least recently seen entries outside this batch.
            idle = sorted((e for e in self.entries.values() if id(e.blocks) not in batch), key=lambda e: e.seen)
            for e in idle[: max(1, len(self.entries) // 4)]:
                del self.entries[id(e.blocks)]
                self.free_rows.append(e.row)
            if not self.free_rows:
                self._grow(2 * self.table.shape[0] + batch_size, 0)
        return self.free_rows.pop()

    def gather(self, tables: Sequence[list], extra: Sequence[int] = ()) -> tuple[torch.Tensor, torch.Tensor]:
        """The (len(tables), width) zero-padded int32 block tables on the
        device, width = the longest table (at least 1), and `extra` (int32) on
        the device, from one transfer."""
        self.step += 1
        n = len(tables)
        width = max(max((len(t) for t in tables), default=0), 1)
        if width > self.table.shape[1]:
            self._grow(0, max(width, 2 * self.table.shape[1]))
        batch = {id(t) for t in tables}
        rows = np.empty(n, dtype=np.int32)
        upd_rows: list[int] = []
        upd_cols: list[int] = []
        upd_vals: list[int] = []
        for i, blocks in enumerate(tables):
            e = self.entries.get(id(blocks))
            if e is None or e.blocks is not blocks:
                e = _Entry(blocks, self._take_row(batch, n))
                self.entries[id(blocks)] = e
            m = len(blocks)
            if m < e.synced or (e.synced and blocks[e.synced - 1] != e.last):
                e.synced = 0  # changed in place: upload it whole
            if e.synced == 0:
                stale = self.row_len[e.row]
                if stale > m:  # clear what a previous owner of the row left past this list
                    upd_rows += [e.row] * (stale - m)
                    upd_cols += range(m, stale)
                    upd_vals += [0] * (stale - m)
            if m > e.synced:
                upd_rows += [e.row] * (m - e.synced)
                upd_cols += range(e.synced, m)
                upd_vals += blocks[e.synced:m]
                self.uploaded += m - e.synced
            if m:
                e.last = blocks[m - 1]
            e.synced = m
            self.row_len[e.row] = m
            e.seen = self.step
            rows[i] = e.row
        k = len(upd_rows)
        payload = np.empty(n + len(extra) + 3 * k, dtype=np.int32)
        payload[:n] = rows
        payload[n:n + len(extra)] = np.asarray(extra, dtype=np.int64)
        if k:
            payload[n + len(extra):] = np.concatenate([np.asarray(upd_rows), np.asarray(upd_cols), np.asarray(upd_vals)])
        host = torch.from_numpy(payload)
        if self.device.type == "cuda":
            host = host.pin_memory()
        dev = host.to(self.device, non_blocking=True)
        if k:
            base = n + len(extra)
            ur, uc, uv = dev[base:base + k].long(), dev[base + k:base + 2 * k].long(), dev[base + 2 * k:]
            self.table.index_put_((ur, uc), uv)
        out = torch.index_select(self.table[:, :width], 0, dev[:n].long())
        return out, dev[n:n + len(extra)]
