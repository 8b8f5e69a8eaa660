"""Speculative round orchestration (ferric_amd/speculative.py) on the CPU,
with deterministic stand-in models: positions, commit ends, anchors and the
draft catch-up follow the reference's index contract
(docs/M1_SPECULATIVE_KV_INDEXING.md; speculative_kv_indexing.rs:498-600), and
the emitted stream equals plain greedy decoding of the target
(speculation.rs:126: greedy speculation never changes the target's output)."""

import numpy as np
import pytest

from ferric_amd import PagedLimits, PagePool
from ferric_amd.runner import BatchOutput
from ferric_amd import FerricError
from ferric_amd.speculative import (SpeculativeDecoder, compact_completion, token_assembly, verify_greedy,
                                      verify_greedy_batch)

VOCAB = 50


class MockRunner:
    """A 'model' whose greedy choice after position p is a hash of the
    tokens written at positions 0..p of the row's sequence. Writes happen
    for every row of a batch before any choice is formed, as on the GPU."""

    def __init__(self, salt):
        self.salt = salt
        self.kv = {}  # (sequence, position) -> token
        self.batches = []

    def choice(self, seq, pos):
        h = self.salt
        for p in range(pos + 1):
            h = (h * 1000003 + self.kv[(seq, p)] + 7) % 2_147_483_647
        return h % VOCAB

    def execute_batch(self, batch, outputs):
        self.batches.append([(r.sequence, r.token, r.position) for r in batch.rows])
        for r in batch.rows:
            self.kv[(r.sequence, r.position)] = r.token
        rows = batch.rows
        return BatchOutput([self.choice(rows[i].sequence, rows[i].position) for i in outputs])


class AgreeingDraft(MockRunner):
    """Draft that agrees with the target except where (seq + pos) % period == 0."""

    def __init__(self, target, period):
        super().__init__(0)
        self.target, self.period = target, period

    def choice(self, seq, pos):
        saved = self.target.kv
        self.target.kv = self.kv
        try:
            c = self.target.choice(seq, pos)
        finally:
            self.target.kv = saved
        return (c + 1) % VOCAB if (seq + pos) % self.period == 0 else c


def plain_greedy(prompt, steps, salt):
    m = MockRunner(salt)
    for p, t in enumerate(prompt):
        m.kv[(1, p)] = t
    out = [m.choice(1, len(prompt) - 1)]
    for i in range(steps):
        m.kv[(1, len(prompt) + i)] = out[-1]
        out.append(m.choice(1, len(prompt) + i))
    return out


def make(k, period):
    limits = PagedLimits(context_tokens=1024, physical_page_count=512, page_table_stride=64)
    target = MockRunner(12345)
    draft = AgreeingDraft(target, period)
    dec = SpeculativeDecoder(target, PagePool(limits, seed=1), draft, PagePool(limits, seed=2), k=k)
    return dec, target, draft


@pytest.mark.parametrize("k,period", [(4, 3), (4, 1000), (1, 2), (3, 5)])
def test_speculative_stream_equals_target_greedy(k, period):
    rng = np.random.default_rng(k * 100 + period)
    prompts = [list(rng.integers(0, VOCAB, n)) for n in (5, 17, 31)]
    dec, target, draft = make(k, period)
    dec.prefill(prompts)
    total_accepted = 0
    for _ in range(12):
        st = dec.round()
        total_accepted += sum(st.accepted)
    for j, p in enumerate(prompts):
        s = dec.seqs[j]
        want = plain_greedy(p, len(s.emitted) - 1, 12345)
        assert s.emitted == want, j
        # committed target KV holds prompt + emitted tokens (the anchor is not yet written)
        hist = list(p) + s.emitted[:-1]
        assert s.cursor == len(hist)
        assert [target.kv[(s.target_sid, i)] for i in range(s.cursor)] == hist
    if period == 1000:
        assert total_accepted == 12 * k * len(prompts)  # the draft always agrees: A = K every round


def test_round_positions_and_commit_ends_follow_the_index_contract():
    dec, target, draft = make(4, 1000)  # full acceptance: exercises the catch-up
    dec.prefill([[1, 2, 3]])
    c0 = dec.seqs[0].cursor
    draft.batches.clear()
    target.batches.clear()
    st = dec.round()
    # draft inputs: anchor at c, candidates at c + 1 .. c + K - 1
    assert [b[0][2] for b in draft.batches] == [c0, c0 + 1, c0 + 2, c0 + 3]
    # target: K + 1 inputs at c .. c + K, anchor first
    assert [r[2] for r in target.batches[0]] == list(range(c0, c0 + 5))
    a = st.accepted[0]
    assert a == 4
    s = dec.seqs[0]
    assert s.cursor == c0 + a + 1  # target commit end
    assert dec.dpool.sequences[s.draft_sid].length == c0 + min(a + 1, 4)  # draft commit end
    assert s.catch_up >= 0
    draft.batches.clear()
    dec.round()
    # the next round starts with the draft catch-up at position c + K
    assert draft.batches[0] == [(s.draft_sid, draft.batches[0][0][1], c0 + 4)]


def test_assembly_and_settlement_match_the_reference_vectors():
    ids = token_assembly([10, 20], np.array([[1, 2], [3, 4]], np.uint32), 2)  # draft[i][s]
    assert ids.tolist() == [[10, 1, 3], [20, 2, 4]]
    assert verify_greedy([3, 4, 5], [9, 4, 5, 6]) == (0, [9])
    assert verify_greedy([3, 4, 5], [3, 4, 9, 6]) == (2, [3, 4, 9])
    assert verify_greedy([3, 4, 5], [3, 4, 5, 6]) == (3, [3, 4, 5, 6])


def test_rounds_carry_compact_completion_records():
    # Each round's 120-byte records (ferric_qwen3_compact_completion_v1,
    # logits.rs:279) name the sequence's slot, the round's epoch and plan, and
    # hold exactly the emitted tokens the settlement produced (the record
    # builder itself is pinned to the reference's vectors in
    # tests/test_compact_record.py).
    import struct

    dec, target, draft = make(4, 3)
    dec.prefill([[1, 2, 3], [4, 5], [6]])
    for epoch in range(5):
        st = dec.round()
        assert len(st.records) == 3
        for s, rec in enumerate(st.records):
            slot, gen, ep = struct.unpack_from("<IIQ", rec, 0)
            assert (slot, gen, ep) == (s, 1, epoch) and rec[16:48] == dec.plan
            a = st.accepted[s]
            assert rec[48] == a and rec[49] == a + 1 == len(st.emitted[s])
            assert list(struct.unpack_from(f"<{a + 1}I", rec, 52)) == st.emitted[s]
            assert rec[52 + 4 * (a + 1):] == bytes(120 - 52 - 4 * (a + 1))


def test_rounds_wider_than_a_record_settle_without_records():
    # K = 17 is past what a completion record holds (16 drafts, 17 emitted
    # tokens): the record builder rejects it, while the round itself, its
    # settlement and both pools' cursors are unaffected.
    k = 17
    draft = np.arange(k * 2, dtype=np.uint32).reshape(k, 2) % VOCAB
    target = np.zeros((2, k + 1), dtype=np.uint32)
    target[0, :] = np.append(draft[:, 0], 7)  # all accepted
    target[1, 0] = (draft[0, 1] + 1) % VOCAB  # first rejected
    acc, em = verify_greedy_batch(draft, target)
    assert acc.tolist() == [k, 0]
    assert em[0].tolist() == list(draft[:, 0]) + [7] and em[1, 0] == target[1, 0]
    with pytest.raises(FerricError) as e:
        compact_completion(target, draft, [k + 1] * 2, [0, 1], [1, 1], [0, 0], [bytes(range(32))] * 2, k + 1, k)
    assert e.value.status == 1
    dec, tgt, drf = make(k, 1000)  # the draft always agrees: every round accepts all 17
    prompts = [[1, 2, 3], [4, 5]]
    dec.prefill(prompts)
    for _ in range(3):
        st = dec.round()
        assert st.records is None
        assert st.accepted == [k, k]
    for j, p in enumerate(prompts):
        s = dec.seqs[j]
        assert s.emitted == plain_greedy(p, len(s.emitted) - 1, 12345)
        assert dec.tpool.sequences[s.target_sid].length == s.cursor
        assert dec.dpool.sequences[s.draft_sid].length == s.cursor - 1  # the catch-up candidate is pending
