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

from .runner import PAGE_TOKENS, PagedLimits, PreparedBatch, PreparedRow, PreparedRows


class SequenceState:
    """A sequence's committed length and its logical-to-physical page list,
    kept as a uint32 array so a prepared row hands it to the C ABI as is."""

    def __init__(self, sequence: int, capacity: int):
        self.sequence = sequence
        self.length = 0  # committed tokens (KV positions 0..length-1 are written)
        self._table = np.zeros(capacity, dtype=np.uint32)
        self._count = 0
        self._view = self._table[:0]  # the reserved pages, re-sliced only when one is added

    @property
    def pages(self) -> np.ndarray:
        return self._view

    def append_page(self, page: int) -> None:
        self._table[self._count] = page
        self._count += 1
        self._view = self._table[: self._count]


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
        # The last decode batch's page-list block: (sequence ids, page counts)
        # -> (tables, offsets, lengths). Equal ids and counts mean equal lists
        # (a sequence's pages are only appended; a released id never returns).
        self._decode_key = None
        self._decode_tables = None

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
        sequence take consecutive positions. Pages are reserved in row order
        (a row whose position starts a page the sequence does not have yet
        takes the next free page). Every row of a sequence sees the
        sequence's full reserved page list, as a read-only snapshot."""
        if len(rows) <= 4:
            return self._prepare_small(rows)
        if len(rows) <= 256:
            batch = self._prepare_decode(rows)
            if batch is not None:
                return batch
            cols = self._prepare_loop(rows)
        else:
            cols = self._prepare_vector(rows)
        states, sid, token, pos, group = cols
        if len(token) and (int(token.min()) < 0 or int(token.max()) > 0xFFFFFFFF):
            raise ValueError("token outside u32")
        lens = np.fromiter([st._count for st in states], dtype=np.int64, count=len(states))
        offs = np.zeros(len(states), dtype=np.int64)
        if len(states) > 1:
            np.cumsum(lens[:-1], out=offs[1:])
        tables = np.concatenate([st._view for st in states]) if states else np.zeros(0, np.uint32)
        writable = tables[offs[group] + pos // PAGE_TOKENS] if len(token) else np.zeros(0, np.uint32)
        prepared = PreparedRows._trusted(sid.astype(np.uint64), token.astype(np.uint32), pos.astype(np.uint32),
                                         writable, tables, offs, lens, group)
        bid = self._next_batch
        self._next_batch += 1
        return PreparedBatch(bid, prepared, self.limits)

    def _prepare_small(self, rows: list) -> PreparedBatch:
        """prepare() for a few rows (a batch-1 decode step): the row loop's
        bookkeeping on Python lists, one small array per column, and a
        lone sequence's page list handed over as a view of its table (the
        entries a view covers never change: pages are only appended)."""
        sequences = self.sequences
        group_of: dict[int, int] = {}
        states, next_pos = [], []
        sid, token, pos, group = [], [], [], []
        for s, t in rows:
            t = int(t)
            if not 0 <= t <= 0xFFFFFFFF:
                raise ValueError("token outside u32")
            g = group_of.get(s)
            if g is None:
                g = group_of[s] = len(states)
                st = sequences[s]
                states.append(st)
                next_pos.append(st.length)
            else:
                st = states[g]
            p = next_pos[g]
            next_pos[g] = p + 1
            if p // PAGE_TOKENS >= st._count:
                self._ensure(st, p + 1)
            sid.append(s)
            token.append(t)
            pos.append(p)
            group.append(g)
        lens = [st._count for st in states]
        offs = [0] * len(states)
        for g in range(1, len(states)):
            offs[g] = offs[g - 1] + lens[g - 1]
        if len(states) == 1:
            tables = states[0]._table[: lens[0]]
        else:
            tables = np.concatenate([st._view for st in states]) if states else np.zeros(0, np.uint32)
        writable = [int(tables[offs[g] + p // PAGE_TOKENS]) for g, p in zip(group, pos)]
        prepared = PreparedRows._trusted(np.array(sid, np.uint64), np.array(token, np.uint32), np.array(pos, np.uint32),
                                         np.array(writable, np.uint32), tables, np.array(offs, np.int64),
                                         np.array(lens, np.int64), np.array(group, np.int64))
        bid = self._next_batch
        self._next_batch += 1
        return PreparedBatch(bid, prepared, self.limits)

    def _prepare_decode(self, rows: list):
        """prepare() for a batch whose rows all belong to different sequences
        (a decode step): one comprehension per column, and the page-list block
        of the previous such batch reused while its sequences and page counts
        are unchanged (15 of every 16 steps). None when a sequence repeats."""
        sequences = self.sequences
        sid = [r[0] for r in rows]
        states = [sequences[s] for s in sid]
        if len(set(sid)) != len(sid):
            return None
        token = [int(r[1]) for r in rows]
        if min(token) < 0 or max(token) > 0xFFFFFFFF:
            raise ValueError("token outside u32")
        pos = [st.length for st in states]
        for st, p in zip(states, pos):
            if p // PAGE_TOKENS >= st._count:
                self._ensure(st, p + 1)
        counts = [st._count for st in states]
        key = (sid, counts)
        if key == self._decode_key:
            tables, offs, lens = self._decode_tables
        else:
            lens = np.array(counts, dtype=np.int64)
            offs = np.zeros(len(counts), dtype=np.int64)
            np.cumsum(lens[:-1], out=offs[1:])
            tables = np.concatenate([st._view for st in states])
            tables.flags.writeable = False
            self._decode_key, self._decode_tables = key, (tables, offs, lens)
        n = len(rows)
        position = np.array(pos, dtype=np.uint32)
        writable = tables[offs + position // PAGE_TOKENS]
        prepared = PreparedRows._trusted(np.array(sid, dtype=np.uint64), np.array(token, dtype=np.uint32), position,
                                         writable, tables, offs, lens, np.arange(n, dtype=np.int64))
        bid = self._next_batch
        self._next_batch += 1
        return PreparedBatch(bid, prepared, self.limits)

    def _prepare_loop(self, rows: list):
        sequences = self.sequences
        group_of: dict[int, int] = {}
        states, next_pos = [], []  # per sequence, in order of first appearance
        sid, token, pos, group = [], [], [], []
        for s, t in rows:
            g = group_of.get(s)
            if g is None:
                g = group_of[s] = len(states)
                st = sequences[s]
                states.append(st)
                next_pos.append(st.length)
            else:
                st = states[g]
            p = next_pos[g]
            next_pos[g] = p + 1
            if p // PAGE_TOKENS >= st._count:
                self._ensure(st, p + 1)
            sid.append(s)
            token.append(int(t))
            pos.append(p)
            group.append(g)
        n = len(rows)
        return (states, np.fromiter(sid, dtype=np.int64, count=n), np.fromiter(token, dtype=np.int64, count=n),
                np.fromiter(pos, dtype=np.int64, count=n), np.fromiter(group, dtype=np.int64, count=n))

    def _prepare_vector(self, rows: list):
        n = len(rows)
        sid = np.fromiter((r[0] for r in rows), dtype=np.int64, count=n)
        token = np.fromiter((int(r[1]) for r in rows), dtype=np.int64, count=n)
        # Sequences in order of first appearance; rank of each row within its
        # sequence gives positions length, length + 1, ...
        order = np.argsort(sid, kind="stable")
        uniq, first, counts = np.unique(sid[order], return_index=True, return_counts=True)
        appear = np.argsort(order[first], kind="stable")  # unique ids by first row
        remap = np.empty(len(uniq), dtype=np.int64)
        remap[appear] = np.arange(len(uniq), dtype=np.int64)
        rank = np.empty(n, dtype=np.int64)
        rank[order] = np.arange(n, dtype=np.int64) - np.repeat(first, counts)
        group = np.empty(n, dtype=np.int64)
        group[order] = np.repeat(remap, counts)
        states = [self.sequences[int(u)] for u in uniq[appear]]  # KeyError for an unknown sequence
        lengths = np.array([st.length for st in states], dtype=np.int64)
        pos = lengths[group] + rank
        # Page reservations happen at the rows that first need a page: the
        # first row of a sequence, or a row entering a page not reserved yet.
        have = np.array([st._count for st in states], dtype=np.int64)
        event = (pos // PAGE_TOKENS >= have[group]) & ((rank == 0) | (pos % PAGE_TOKENS == 0))
        for i in np.nonzero(event)[0]:
            self._ensure(states[group[i]], int(pos[i]) + 1)
        return states, sid, token, pos, group

    def commit(self, batch: PreparedBatch) -> None:
        rows = batch.rows
        if isinstance(rows, PreparedRows):
            for s, p in zip(rows.sequence.tolist(), rows.position.tolist()):
                st = self.sequences[s]
                st.length = max(st.length, p + 1)
            return
        for r in rows:
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
