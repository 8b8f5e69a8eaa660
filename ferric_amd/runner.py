"""Host-side mirror of the reference's batch-runner boundary.

`TpBatchRunner` has the method set of the reference's
`EngineeringTpBatchRunnerV2` (adapters/m1-engineering-execution-v1/src/
tp_batch_runtime.rs:20-95): `row_capacity`, `execute_batch(batch,
output_rows) -> BatchOutput{choices}`, `output_head_rows`,
`expected_dispatch_counts_for_selection` / `_for_batch`, `dispatch_counts`,
`close`. The prepared-batch
types mirror `EngineeringTpPreparedRowV1` / `EngineeringTpPreparedBatchV1`
(tp_paged.rs:257-350). All GPU work and all batch validation happen in
libferric_hip.so behind the C ABI; this module only marshals.
"""

from __future__ import annotations

import ctypes
from collections.abc import Sequence as _SequenceABC
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np

from . import _lib
from ._lib import FerricError, check, load

PAGE_TOKENS = 16

# Admitted Qwen3 shapes (crates/ferric-spec/src/configuration.rs:107-194).
QWEN3_8B = dict(layers=36, hidden=4096, query_heads=32, kv_heads=8, head_dim=128, intermediate=12288,
                vocabulary=151936, tied_embedding=0, rope_theta=1_000_000, rms_epsilon=1e-6)
QWEN3_0_6B = dict(layers=28, hidden=1024, query_heads=16, kv_heads=8, head_dim=128, intermediate=3072,
                  vocabulary=151936, tied_embedding=1, rope_theta=1_000_000, rms_epsilon=1e-6)


@dataclass(frozen=True)
class PagedLimits:
    """Resident envelope (EngineeringTpPagedLimitsV1)."""

    context_tokens: int
    physical_page_count: int
    page_table_stride: int


@dataclass(frozen=True)
class PreparedRow:
    """One sealed row (EngineeringTpPreparedRowV1)."""

    sequence: int
    token: int
    position: int
    physical_pages: Sequence[int]  # tuple, list or uint32 array
    writable_physical_page: int

    @property
    def writable_token_offset(self) -> int:
        return self.position % PAGE_TOKENS


class PreparedRows(_SequenceABC):
    """The rows of a prepared batch as columns: one entry per row for the
    sequence, token, position and writable page, plus one page list per
    sequence, all of them in one read-only uint32 buffer (`tables`, list g
    at `table_offset[g]`, `table_len[g]` entries) that the sequence's rows
    share (`table_index` picks the list). Indexing or iterating yields
    PreparedRow objects, so it reads like a list of rows; the runner hands
    the columns to the C ABI without a per-row loop."""

    def __init__(self, sequence, token, position, writable, tables, table_offset, table_len, table_index):
        token = np.asarray(token)
        if token.size and (token.min() < 0 or token.max() > 0xFFFFFFFF):
            raise ValueError("token outside u32")
        self.sequence = np.asarray(sequence, dtype=np.uint64)
        self.token = token.astype(np.uint32)
        self.position = np.asarray(position, dtype=np.uint32)
        self.writable = np.asarray(writable, dtype=np.uint32)
        self.tables = np.ascontiguousarray(tables, dtype=np.uint32)
        self.tables.flags.writeable = False
        self.table_offset = np.asarray(table_offset, dtype=np.int64)
        self.table_len = np.asarray(table_len, dtype=np.int64)
        self.table_index = np.asarray(table_index, dtype=np.int64)

    @classmethod
    def _trusted(cls, sequence, token, position, writable, tables, table_offset, table_len, table_index):
        """The same object from columns that already have the final dtypes
        (uint64 sequence, uint32 token/position/writable/tables, int64
        offsets, lengths and indices) and token ids the caller checked: the
        page pool's path, which runs once per decode step."""
        self = cls.__new__(cls)
        self.sequence, self.token, self.position, self.writable = sequence, token, position, writable
        tables.flags.writeable = False
        self.tables, self.table_offset, self.table_len, self.table_index = tables, table_offset, table_len, table_index
        return self

    def __len__(self) -> int:
        return len(self.token)

    def _row(self, i: int) -> PreparedRow:
        g = self.table_index[i]
        off = int(self.table_offset[g])
        return PreparedRow(int(self.sequence[i]), int(self.token[i]), int(self.position[i]),
                           self.tables[off:off + int(self.table_len[g])], int(self.writable[i]))

    def __getitem__(self, i):
        if isinstance(i, slice):
            return [self._row(j) for j in range(*i.indices(len(self)))]
        if i < 0:
            i += len(self)
        if not 0 <= i < len(self):
            raise IndexError("row index out of range")
        return self._row(i)

    def __iter__(self):
        return (self._row(i) for i in range(len(self)))


@dataclass
class PreparedBatch:
    """Move-only batch metadata (EngineeringTpPreparedBatchV1)."""

    id: int
    rows: list
    limits: PagedLimits


@dataclass
class BatchOutput:
    """EngineeringTpBatchOutputV2: one greedy choice per requested output row."""

    choices: list = field(default_factory=list)


def model_desc(cfg: dict) -> _lib.ModelDesc:
    return _lib.ModelDesc(cfg["layers"], cfg["hidden"], cfg["query_heads"], cfg["kv_heads"], cfg["head_dim"],
                          cfg["intermediate"], cfg["vocabulary"], cfg["tied_embedding"], cfg["rope_theta"],
                          cfg["rms_epsilon"])


# fh_row as a numpy record (layout checked against ctypes in the ABI tests).
ROW_DTYPE = np.dtype([("sequence", "<u8"), ("token", "<u4"), ("position", "<u4"), ("pages", "<u8"),
                      ("page_count", "<u4"), ("writable_page", "<u4")])


class _RowWords(ctypes.Structure):
    """fh_row with the page list as a plain address (same layout as _lib.Row)."""

    _fields_ = [("sequence", ctypes.c_uint64), ("token", ctypes.c_uint32), ("position", ctypes.c_uint32),
                ("pages", ctypes.c_uint64), ("page_count", ctypes.c_uint32), ("writable_page", ctypes.c_uint32)]


_SMALL_BATCH = 4  # rows up to which a batch is marshalled field by field (cheaper than column copies)


def _rows_to_c(rows: Sequence[PreparedRow]):
    """fh_row[] for the C ABI; returns (pointer, objects that must stay alive)."""
    n = len(rows)
    if isinstance(rows, PreparedRows) and 0 < n <= _SMALL_BATCH:
        arr = (_RowWords * n)()
        base = rows.tables.__array_interface__["data"][0]
        seq, tok, pos, wr = rows.sequence.tolist(), rows.token.tolist(), rows.position.tolist(), rows.writable.tolist()
        grp, offs, lens = rows.table_index.tolist(), rows.table_offset.tolist(), rows.table_len.tolist()
        for i in range(n):
            r, g = arr[i], grp[i]
            r.sequence, r.token, r.position, r.writable_page = seq[i], tok[i], pos[i], wr[i]
            r.page_count = lens[g]
            r.pages = base + 4 * offs[g] if lens[g] else 0
        return ctypes.cast(arr, ctypes.POINTER(_lib.Row)), [arr, rows.tables]
    rec = np.zeros(max(n, 1), dtype=ROW_DTYPE)
    keep = [rec]
    if isinstance(rows, PreparedRows):
        keep.append(rows.tables)
        if n:
            base = rows.tables.ctypes.data if len(rows.tables) else 0
            lens = rows.table_len[rows.table_index]
            rec["sequence"][:n] = rows.sequence
            rec["token"][:n] = rows.token
            rec["position"][:n] = rows.position
            rec["pages"][:n] = np.where(lens > 0, base + 4 * rows.table_offset[rows.table_index], 0).astype(np.uint64)
            rec["page_count"][:n] = lens
            rec["writable_page"][:n] = rows.writable
        return ctypes.cast(rec.ctypes.data, ctypes.POINTER(_lib.Row)), keep
    seq, tok, pos, ptrs, cnt, wp = [], [], [], [], [], []
    converted = {}  # id(page list) -> (array, pointer): rows of a sequence share one list
    for r in rows:
        pages = r.physical_pages
        hit = converted.get(id(pages))
        if hit is None or hit[2] is not pages:
            arr = _page_array(pages)
            hit = (arr, arr.ctypes.data if len(arr) else 0, pages)
            converted[id(pages)] = hit
            keep.append(arr)
        seq.append(r.sequence)
        tok.append(r.token)
        pos.append(r.position)
        ptrs.append(hit[1])
        cnt.append(len(hit[0]))
        wp.append(r.writable_physical_page)
    if n:
        rec["sequence"][:n] = seq
        rec["token"][:n] = tok
        rec["position"][:n] = pos
        rec["pages"][:n] = ptrs
        rec["page_count"][:n] = cnt
        rec["writable_page"][:n] = wp
    return ctypes.cast(rec.ctypes.data, ctypes.POINTER(_lib.Row)), keep


def _page_array(pages) -> np.ndarray:
    if isinstance(pages, np.ndarray) and pages.dtype == np.uint32 and pages.flags.c_contiguous:
        return pages
    return np.ascontiguousarray(np.asarray(pages, dtype=np.uint32))


class TpBatchRunner:
    """One-GPU runner behind the reference's batch-runner boundary."""

    def __init__(self, model: dict, limits: PagedLimits, row_capacity: int = 32, use_graphs: bool = True,
                 capture_hidden: bool = False, device: int = 0, prefill_rows: int = 0):
        self._lib = load()
        self.model = dict(model)
        self.limits = limits
        self._desc = model_desc(model)
        self._opts = _lib.CtxOptions(row_capacity, limits.physical_page_count, limits.page_table_stride,
                                     limits.context_tokens, 1 if use_graphs else 0, 1 if capture_hidden else 0,
                                     device, prefill_rows)
        ctx = ctypes.c_void_p()
        st = self._lib.fh_create(ctypes.byref(self._desc), ctypes.byref(self._opts), ctypes.byref(ctx))
        check(st, None, "fh_create")
        self._ctx = ctx
        self._rows_last = 0  # rows with logits in the last batch
        self._batch_rows_last = 0  # token rows of the last batch

    # ---- reference boundary ----
    def row_capacity(self) -> int:
        return int(self._lib.fh_row_capacity(self._ctx))

    def execute_batch(self, batch: PreparedBatch, output_rows: Sequence[int]) -> BatchOutput:
        if batch.limits != self.limits:
            raise FerricError(2, "foreign, stale, or invalid prepared GPU batch")
        rows, keep = _rows_to_c(batch.rows)
        outs = np.ascontiguousarray(np.asarray(output_rows, dtype=np.uint32))
        choices = np.zeros(max(len(outs), 1), dtype=np.uint32)
        st = self._lib.fh_execute_batch(self._ctx, batch.id, rows, len(batch.rows),
                                        outs.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(outs),
                                        choices.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
        del keep
        check(st, self._ctx)
        # Decode batches produce logits for every row, prefill chunks for the output rows only.
        self._rows_last = len(batch.rows) if len(batch.rows) <= self._opts.row_capacity else len(outs)
        self._batch_rows_last = len(batch.rows)
        return BatchOutput([int(c) for c in choices[: len(outs)]])

    def output_head_rows(self, physical: int, published: int) -> int:
        return physical

    def expected_dispatch_counts_for_selection(self, batch: PreparedBatch, output_rows: Sequence[int]) -> list:
        """The dispatch_counts() increment execute_batch(batch, output_rows) will
        make (one entry: one context stands in for every rank), evaluated by
        the library without launching (fh_expected_dispatch_count). Raises the
        execute_batch error for a batch it would reject."""
        if batch.limits != self.limits:
            raise FerricError(2, "foreign, stale, or invalid prepared GPU batch")
        rows, keep = _rows_to_c(batch.rows)
        outs = np.ascontiguousarray(np.asarray(output_rows, dtype=np.uint32))
        count = ctypes.c_uint64()
        st = self._lib.fh_expected_dispatch_count(self._ctx, batch.id, rows, len(batch.rows),
                                                  outs.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(outs),
                                                  ctypes.byref(count))
        del keep
        check(st, self._ctx)
        return [int(count.value)]

    def expected_dispatch_counts_for_batch(self, batch: PreparedBatch, published: int) -> list:
        """As the reference's default: the selection of the first `published` rows."""
        return self.expected_dispatch_counts_for_selection(batch, range(published))

    def expected_dispatch_counts(self, published: int) -> list:
        """The batch-independent form has no exact answer here: the launch
        schedule depends on the batch (rows, written slots, prefill or decode).
        Use expected_dispatch_counts_for_selection."""
        raise FerricError(1, "the dispatch count depends on the batch; use expected_dispatch_counts_for_selection")

    def dispatch_counts(self) -> list:
        return [int(self._lib.fh_dispatch_count(self._ctx))]

    def close(self) -> None:
        if self._ctx:
            self._lib.fh_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- setup ----
    def upload_weight(self, kind: int, layer: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data, dtype=np.uint16).reshape(-1)
        st = self._lib.fh_upload_weight(self._ctx, kind, layer, data.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                                        data.size)
        check(st, self._ctx)

    def download_weight(self, kind: int, layer: int, elements: int) -> np.ndarray:
        out = np.zeros(elements, dtype=np.uint16)
        check(self._lib.fh_download_weight(self._ctx, kind, layer, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                                           elements), self._ctx)
        return out

    def synthesize_weights(self, seed: int, sigma: float = 0.02) -> None:
        check(self._lib.fh_synthesize_weights(self._ctx, seed, sigma), self._ctx)

    def kv_fill_synthetic(self, seed: int, sigma: float, rows: Sequence[PreparedRow], keys: Sequence[int],
                          context_stride: int) -> None:
        crow, keep = _rows_to_c(rows)
        k = np.ascontiguousarray(np.asarray(keys, dtype=np.uint64))
        st = self._lib.fh_kv_fill_synthetic(self._ctx, seed, sigma, crow, k.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                                            len(rows), context_stride)
        del keep
        check(st, self._ctx)

    # ---- parity readbacks ----
    def read_logits(self) -> np.ndarray:
        n = self._rows_last * self.model["vocabulary"]
        out = np.zeros(n, dtype=np.float32)
        check(self._lib.fh_read_logits(self._ctx, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n), self._ctx)
        return out.reshape(self._rows_last, self.model["vocabulary"])

    def read_hidden(self, layer: int) -> np.ndarray:
        """Residual stream after `layer` for every token row of the last batch."""
        n = self._batch_rows_last * self.model["hidden"]
        out = np.zeros(n, dtype=np.uint16)
        check(self._lib.fh_read_hidden(self._ctx, layer, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), n),
              self._ctx)
        return out.reshape(self._batch_rows_last, self.model["hidden"])

    def read_kv_page(self, layer: int, which: int, page: int) -> np.ndarray:
        n = PAGE_TOKENS * self.model["kv_heads"] * 128
        out = np.zeros(n, dtype=np.uint16)
        check(self._lib.fh_read_kv_page(self._ctx, layer, which, page,
                                        out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), n), self._ctx)
        return out

    def read_kv_cache(self, layer: int, which: int) -> np.ndarray:
        """One layer's whole K (which = 0) or V (1) pool, [pages * 16 * kv_heads * 128] bf16."""
        n = self.limits.physical_page_count * PAGE_TOKENS * self.model["kv_heads"] * 128
        out = np.zeros(n, dtype=np.uint16)
        check(self._lib.fh_read_kv_cache(self._ctx, layer, which, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                                         n), self._ctx)
        return out

    def write_kv_page(self, layer: int, which: int, page: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data, dtype=np.uint16)
        check(self._lib.fh_write_kv_page(self._ctx, layer, which, page,
                                         data.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), data.size), self._ctx)

    # ---- timing ----
    def last_step_ms(self) -> float:
        return float(self._lib.fh_last_step_ms(self._ctx))

    def set_profiling(self, enabled: bool) -> None:
        check(self._lib.fh_set_profiling(self._ctx, 1 if enabled else 0), self._ctx)

    def time_attention(self, reps: int = 20) -> float:
        """Mean ms of the last decode batch's attention launch, re-run back to back."""
        ms = ctypes.c_float()
        check(self._lib.fh_time_attention(self._ctx, reps, ctypes.byref(ms)), self._ctx)
        return float(ms.value)

    def kernel_class_ms(self) -> dict:
        out = {}
        for i, name in enumerate(_lib.KERNEL_CLASSES):
            ms = ctypes.c_float()
            n = ctypes.c_uint32()
            check(self._lib.fh_kernel_class_ms(self._ctx, i, ctypes.byref(ms), ctypes.byref(n)), self._ctx)
            out[name] = (float(ms.value), int(n.value))
        return out
