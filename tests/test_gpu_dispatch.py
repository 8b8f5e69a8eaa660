"""The dispatch preflight against the launches a batch really issues.

The reference's runtime asks the runner, before each submission, for the
dispatch-count increment the batch will make
(expected_dispatch_counts_for_selection, tp_batch_runtime.rs:80-86) and
rejects the batch when dispatch_counts() moved by anything else
(tp_batch_runtime.rs:432-446). Here fh_expected_dispatch_count must equal the
fh_dispatch_count increment for every schedule the library has: decode steps of
7, 8 or 9 launches per layer, graph replays of different graph keys in turn,
prefill chunks of both kinds, and capture runs. Contents do not matter for the
count (the policy reads the shape, the context envelope and which rows read
other rows' new slots), so every batch starts near position 0.
"""

from __future__ import annotations

import pytest

import ferric_amd
from ferric_amd import PagedLimits, PagePool, TpBatchRunner

pytestmark = pytest.mark.gpu

L8 = ferric_amd.QWEN3_8B["layers"]
L06 = ferric_amd.QWEN3_0_6B["layers"]


def decode_launches(layers, qk_in_attention, merge_in_attention, capture=False, one_row=False):
    """Launches of a decode step: metadata ingest + embedding; per layer RMSNorm,
    QKV, [QK-norm/RoPE/KV append], attention partitions, [merge], O, RMSNorm,
    gate/up, down; final norm, head, two argmax passes; one copy per layer
    when the residual stream is captured. One row: the three norms run inside
    the QKV, gate/up and head launches."""
    per_layer = 7 + (0 if qk_in_attention else 1) + (0 if merge_in_attention else 1)
    norms = 2 * layers + 1 if one_row else 0
    return 5 + layers * per_layer + (layers if capture else 0) - norms


def prefill_launches(layers, rows, outputs, private=True):
    """Launches of a prefill chunk: clear, embedding; per layer the chunk's
    schedule (over 256 rows: norm, QKV with the QK-norm in its epilogue,
    attention, O + residual, norm, gate/up, down + residual; up to 256 rows:
    split-K partials folded by the norms, the input norm launched once, and,
    where no attention block reads a slot another block writes (`private`),
    the QK-norm inside the attention launch); then gather, final norm, head
    and two argmax passes for the output rows."""
    head = 5 if outputs else 0
    if rows > 256:
        return 2 + 7 * layers + head
    return 2 + 1 + (7 if private else 8) * layers + head


def run_checked(runner, pool, rows, outs=None, expect=None):
    batch = pool.prepare(rows)
    outs = list(range(len(rows))) if outs is None else outs
    (pre,) = runner.expected_dispatch_counts_for_selection(batch, outs)
    (before,) = runner.dispatch_counts()
    runner.execute_batch(batch, outs)
    (after,) = runner.dispatch_counts()
    pool.commit(batch)
    print(f"{len(rows)} rows, {len(outs)} outputs: expected {pre}, issued {after - before}", flush=True)
    assert after - before == pre
    if expect is not None:
        assert pre == expect
    return pre


@pytest.fixture(scope="module")
def runner8b():
    # The 8B model at the batch-32 workload's context envelope (8192 + headroom
    # tokens): the merge policy depends on that envelope, not on the positions.
    ctx = 8192 + 128
    limits = PagedLimits(context_tokens=ctx, physical_page_count=640, page_table_stride=ctx // 16)
    runner = TpBatchRunner(ferric_amd.QWEN3_8B, limits, row_capacity=32, use_graphs=True, prefill_rows=280)
    runner.synthesize_weights(5, 0.02)
    # One pool for the module: batch ids must keep increasing on one runner.
    yield runner, PagePool(limits, seed=1)
    runner.close()


def test_8b_decode_graph_keys_in_turn(runner8b):
    runner, pool = runner8b
    wide = [pool.admit(0) for _ in range(32)]
    one = pool.admit(0)
    rows32 = lambda t: [(s, t + i) for i, s in enumerate(wide)]
    # 32 rows: QK-norm launch and merge launch of their own.
    b32 = decode_launches(L8, False, False)
    # One row: both inside the attention launch, the norms inside the projections.
    b1 = decode_launches(L8, True, True, one_row=True)
    assert (b32, b1) == (329, 184)
    for step in range(3):
        # Capture, replay, and replays of the other graph key in between.
        run_checked(runner, pool, rows32(10 * step), expect=b32)
        run_checked(runner, pool, [(one, 100 + step)], expect=b1)


def test_8b_small_and_same_sequence_batches(runner8b):
    runner, pool = runner8b
    four = [pool.admit(0) for _ in range(4)]
    # Four rows of four sequences: 4 x 8 KV heads x 17 partitions <= 1024, so
    # the partitions merge inside the attention launch, and every written slot
    # is private, so the QK-norm/KV append runs there too.
    run_checked(runner, pool, [(s, 7) for s in four], expect=decode_launches(L8, True, True))
    # Three rows of one sequence: each row reads the slots the rows before it
    # write, so the QK-norm/KV append keeps its own launch.
    seq = pool.admit(0)
    run_checked(runner, pool, [(seq, 1), (seq, 2), (seq, 3)], expect=decode_launches(L8, False, True))
    # The same batches again, now replayed from their graphs.
    run_checked(runner, pool, [(s, 8) for s in four], expect=decode_launches(L8, True, True))
    run_checked(runner, pool, [(seq, 4), (seq, 5), (seq, 6)], expect=decode_launches(L8, False, True))


def test_8b_prefill_chunks(runner8b):
    runner, pool = runner8b
    # 280 rows: 7 prompts of 40 tokens, the last token of each an output row.
    sids = [pool.admit(0) for _ in range(7)]
    rows = [(s, 11 + t) for s in sids for t in range(40)]
    run_checked(runner, pool, rows, outs=[40 * i + 39 for i in range(7)], expect=prefill_launches(L8, 280, 7))
    # 42 rows (the split-K panel path), then a chunk without output rows.
    sids = [pool.admit(0) for _ in range(3)]
    rows = [(s, 5 + t) for s in sids for t in range(14)]
    run_checked(runner, pool, rows, outs=[13, 27, 41], expect=prefill_launches(L8, 42, 3))
    sids = [pool.admit(0) for _ in range(3)]
    rows = [(s, 5 + t) for s in sids for t in range(14)]
    run_checked(runner, pool, rows, outs=[], expect=prefill_launches(L8, 42, 0))
    # 42 rows of one sequence: three attention blocks, the later ones reading
    # the pages the earlier ones write, so the QK-norm keeps its own launch.
    seq = pool.admit(0)
    rows = [(seq, 3 + t) for t in range(42)]
    run_checked(runner, pool, rows, outs=[41], expect=prefill_launches(L8, 42, 1, private=False))


def test_0_6b_batch32_and_capture():
    ctx = 2048 + 64
    limits = PagedLimits(context_tokens=ctx, physical_page_count=256, page_table_stride=ctx // 16)
    for capture in (False, True):
        runner = TpBatchRunner(ferric_amd.QWEN3_0_6B, limits, row_capacity=32, use_graphs=not capture,
                               capture_hidden=capture)
        try:
            runner.synthesize_weights(6, 0.02)
            pool = PagePool(limits, seed=4)
            sids = [pool.admit(0) for _ in range(32)]
            # 16 query heads: QK-norm inside attention at any size; 32 x 8 x 9
            # partitions > 1024, so the merge has its own launch.
            expect = decode_launches(L06, True, False, capture=capture)
            if not capture:
                assert expect == 229
            for step in range(2):
                run_checked(runner, pool, [(s, 3 + step) for s in sids], expect=expect)
            # One row: the norms inside the QKV, gate/up and head launches; the
            # capture copies read the residual stream's current buffer.
            one = decode_launches(L06, True, True, capture=capture, one_row=True)
            assert one == (144 + 28 if capture else 144)
            for step in range(2):
                run_checked(runner, pool, [(sids[0], 5 + step)], expect=one)
        finally:
            runner.close()


def test_preflight_rejects_what_execute_rejects(runner8b):
    runner, pool = runner8b
    s = pool.admit(0)
    batch = pool.prepare([(s, 1)])
    with pytest.raises(ferric_amd.FerricError) as e:
        runner.expected_dispatch_counts_for_selection(batch, [1])
    assert e.value.status == 5  # output rows outside the batch
    with pytest.raises(ferric_amd.FerricError):
        runner.expected_dispatch_counts(1)
