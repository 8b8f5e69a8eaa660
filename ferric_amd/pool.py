"""A minimal caller-side page pool, for tests and the benchmark.

The reference's pool and scheduler (EngineeringTpPagedPoolV1 /
EngineeringTpBatchRuntimeV2, adapters/m1-engineering-execution-v1/src/
tp_paged.rs:643 and tp_batch_runtime.rs:314-480) sit *above* the runner
boundary and are not part of this library. This stand-in plays their role:
it owns physical page ids (a seeded, shuffled free list), gives each sequence a
logical-to-physical page list, reserves the page that holds each row's write
slot before the call, and commits lengths after a successful step.
"""

from __future__ import annotations

import random

import numpy as np

from .runner import PAGE_TOKENS, PagedLimits, PreparedBatch, PreparedRow


class SequenceState:
    """A sequence's committed length and its logical-to-physical page list,
    kept as a uint32 array so a prepared row hands it to the C ABI as is."""

    def __init__(self, sequence: int, capacity: int):
        self.sequence = sequence
        self.length = 0  # committed tokens (KV positions 0..length-1 are written)
        self._table = np.zeros(capacity, dtype=np.uint32)
        self._count = 0

    @property
    def pages(self) -> np.ndarray:
        return self._table[: self._count]

    def append_page(self, page: int) -> None:
        self._table[self._count] = page
        self._count += 1


class PagePool:
    def __init__(self, limits: PagedLimits, seed: int = 0, shuffle: bool = True):
        self.limits = limits
        free = list(range(limits.physical_page_count))
        if shuffle:
            random.Random(seed).shuffle(free)
        self.free = free
        self.sequences: dict[int, SequenceState] = {}
        self._next_seq = 1
        self._next_batch = 1

    def admit(self, prefix_tokens: int = 0) -> int:
        """Admits a sequence whose first `prefix_tokens` KV positions are already resident."""
        sid = self._next_seq
        self._next_seq += 1
        st = SequenceState(sid, self.limits.page_table_stride)
        self._ensure(st, prefix_tokens)
        st.length = prefix_tokens
        self.sequences[sid] = st
        return sid

    def _ensure(self, st: SequenceState, tokens: int) -> None:
        need = (tokens + PAGE_TOKENS - 1) // PAGE_TOKENS
        if need > self.limits.page_table_stride:
            raise ValueError("sequence exceeds the page-table stride")
        while len(st.pages) < need:
            if not self.free:
                raise MemoryError("out of KV pages")
            st.append_page(self.free.pop())

    def prepare(self, rows: list) -> PreparedBatch:
        """rows: [(sequence, token)] in scheduler order; consecutive rows of one
        sequence take consecutive positions."""
        pending: dict[int, int] = {}
        prepared = []
        for sid, token in rows:
            st = self.sequences[sid]
            pos = st.length + pending.get(sid, 0)
            pending[sid] = pending.get(sid, 0) + 1
            self._ensure(st, pos + 1)
            prepared.append((sid, int(token), pos, int(st.pages[pos // PAGE_TOKENS])))
        # Every row of a sequence sees the sequence's full reserved page list
        # (a read-only copy: later growth of the sequence does not change it).
        tables = {}
        for sid in pending:
            t = self.sequences[sid].pages.copy()
            t.flags.writeable = False
            tables[sid] = t
        prepared = [PreparedRow(sid, token, pos, tables[sid], page) for sid, token, pos, page in prepared]
        bid = self._next_batch
        self._next_batch += 1
        return PreparedBatch(bid, prepared, self.limits)

    def commit(self, batch: PreparedBatch) -> None:
        for r in batch.rows:
            st = self.sequences[r.sequence]
            st.length = max(st.length, r.position + 1)

    def truncate(self, sid: int, length: int) -> None:
        """Commits a sequence to exactly `length` tokens: positions from
        `length` on are a rejected suffix (written, unpublished, rewritten by
        the next step). Reserved pages stay with the sequence."""
        st = self.sequences[sid]
        if length < 0 or (length + PAGE_TOKENS - 1) // PAGE_TOKENS > len(st.pages):
            raise ValueError("commit end outside the reserved pages")
        st.length = length

    def release(self, sid: int) -> None:
        st = self.sequences.pop(sid)
        self.free.extend(int(p) for p in st.pages)
