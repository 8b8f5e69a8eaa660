"""Greedy speculative decoding over two runners (a draft and a target model).

Host orchestration of one speculative round with the reference's index
contract (docs/M1_SPECULATIVE_KV_INDEXING.md; crates/ferric-spec/src/
speculative_kv_indexing.rs:498-600) and greedy settlement
(crates/ferric-spec/src/speculation.rs:126-200). For a round of width K at
the shared cursor c with round anchor a (the last emitted token, not yet in
either KV cache):

  * draft: K decode steps; input 0 is a at position c, input i is the
    candidate d[i-1] at position c + i; step i's choice is candidate d[i];
  * target: one batch with the K + 1 inputs [a, d[0] .. d[K-1]] of every
    sequence at positions c .. c + K (the token assembly of
    ferric_qwen3_speculative_token_assembly_v1, logits.rs:587); choice i is
    the target's greedy token after input i;
  * settle: A = longest prefix with d[i] == t[i]; emitted = d[0..A) + t[A];
  * commit: target to c + A + 1, draft to c + min(A + 1, K); the rest of
    each tentative interval is a rejected suffix. t[A] is the next anchor.
    When A == K the draft never consumed d[K-1]: the next round first runs
    a draft catch-up step with d[K-1] at position c + K.

The integer work (assembly, settlement, the per-sequence 120-byte
completion record of ferric_qwen3_compact_completion_v1, logits.rs:279)
runs through the C ABI (fh_speculative_token_assembly,
fh_verify_greedy_round, fh_compact_completion).
"""

from __future__ import annotations

import ctypes
import hashlib
from dataclasses import dataclass

import numpy as np

from ._lib import check, load
from .pool import PagePool
from .runner import TpBatchRunner


@dataclass
class SpecSequence:
    target_sid: int
    draft_sid: int
    cursor: int  # committed tokens of the target (= the draft once caught up)
    anchor: int  # last emitted token, not yet processed by either model
    catch_up: int = -1  # draft candidate still to be consumed at cursor - 1, or -1
    emitted: list = None


@dataclass
class RoundStats:
    accepted: list
    emitted: list
    draft_steps: int
    catch_up_rows: int
    target_rows: int
    records: list = None  # one 120-byte completion record per sequence (bytes)
    draft: np.ndarray = None  # the round's draft choices, iteration-major [K][S]
    target_choices: np.ndarray = None  # the verify batch's choices [S][K + 1]


def _u32(a):
    a = np.ascontiguousarray(np.asarray(a, dtype=np.uint32))
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))


def token_assembly(anchors, draft_iteration_major, k):
    """target_ids[s][0] = anchors[s], target_ids[s][1 + i] = draft[i][s]."""
    lib = load()
    s = len(anchors)
    a, ap = _u32(anchors)
    d, dp = _u32(np.asarray(draft_iteration_major, dtype=np.uint32).reshape(-1) if k else [0])
    out = np.zeros(s * (k + 1), dtype=np.uint32)
    check(lib.fh_speculative_token_assembly(ap, dp if k else None, s, k,
                                            out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))))
    return out.reshape(s, k + 1)


def verify_greedy(draft, target):
    """(accepted, emitted) of speculation.rs:126 for one sequence."""
    lib = load()
    d, dp = _u32(draft)
    t, tp = _u32(target)
    acc = ctypes.c_uint32()
    em = (ctypes.c_uint32 * (len(draft) + 1))()
    n = ctypes.c_uint32()
    check(lib.fh_verify_greedy_round(dp if len(draft) else None, len(draft), tp, len(target), ctypes.byref(acc), em,
                                     ctypes.byref(n)))
    return int(acc.value), [int(x) for x in em[: n.value]]


def verify_greedy_batch(draft_iteration_major, target):
    """verify_greedy for every sequence of a round in one C call: draft [K][S],
    target [S][K + 1]; returns (accepted [S], emitted [S][K + 1]) with the
    first accepted[s] + 1 entries of emitted[s] meaningful."""
    lib = load()
    t, tp = _u32(np.asarray(target, dtype=np.uint32).reshape(-1))
    s = int(np.asarray(target).shape[0])
    k = t.size // s - 1 if s else 0
    d, dp = _u32(np.asarray(draft_iteration_major, dtype=np.uint32).reshape(-1) if k else [0])
    accepted = np.zeros(max(s, 1), dtype=np.uint32)
    emitted = np.zeros(max(s * (k + 1), 1), dtype=np.uint32)
    check(lib.fh_verify_greedy_batch(dp if k else None, tp, s, k,
                                     accepted.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                     emitted.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))))
    return accepted[:s], emitted[: s * (k + 1)].reshape(s, k + 1)


def compact_completion(choices, draft, active_lengths, slots, generations, epochs, plans, active_tokens, k):
    """Per-sequence completion records (list of 120-byte strings) of
    fh_compact_completion: choices [S][active_tokens], draft [K][S]
    (iteration-major), plans: S 32-byte plan identities."""
    lib = load()
    s = len(active_lengths)
    c, cp = _u32(np.asarray(choices, dtype=np.uint32).reshape(-1))
    d, dp = _u32(np.asarray(draft, dtype=np.uint32).reshape(-1) if k else [0])
    lv, lp = _u32(active_lengths)
    sl, sp = _u32(slots)
    gn, gp = _u32(generations)
    ep = np.ascontiguousarray(np.asarray(epochs, dtype=np.uint64))
    pl = np.frombuffer(b"".join(bytes(p) for p in plans), dtype=np.uint8).copy()
    if pl.size != 32 * s:
        raise ValueError("one 32-byte plan identity per sequence")
    out = np.zeros(s * 120, dtype=np.uint8)
    u8 = ctypes.POINTER(ctypes.c_uint8)
    check(lib.fh_compact_completion(cp, dp if k else None, lp, sp, gp, ep.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                                    pl.ctypes.data_as(u8), s, active_tokens, k, out.ctypes.data_as(u8)))
    return [bytes(out[i * 120:(i + 1) * 120]) for i in range(s)]


# Limits of the 120-byte completion record (logits.rs:279): at most 32
# request slots, 16 draft tokens (17 emitted), token ids below 151936.
RECORD_MAX_SEQUENCES = 32
RECORD_MAX_K = 16
RECORD_VOCABULARY = 151936


def round_records(choices, draft, k, epoch, plan):
    """The completion records of a settled round (slot = sequence index,
    generation 1, epoch = round), or None where the round is outside what a
    record can hold (more than 32 sequences, K > 16, or a token id a record
    rejects); the round itself is unaffected."""
    choices, draft = np.asarray(choices), np.asarray(draft)
    n = int(choices.shape[0])
    if n == 0 or n > RECORD_MAX_SEQUENCES or k > RECORD_MAX_K:
        return None
    if int(choices.max()) >= RECORD_VOCABULARY or (draft.size and int(draft.max()) >= RECORD_VOCABULARY):
        return None
    return compact_completion(choices, draft, [k + 1] * n, list(range(n)), [1] * n, [epoch] * n, [plan] * n, k + 1,
                              k)


class SpeculativeDecoder:
    """Greedy speculation of a draft runner for a target runner, each with
    its own KV pool. Sequences share prompts and cursors across the two."""

    def __init__(self, target: TpBatchRunner, target_pool: PagePool, draft: TpBatchRunner, draft_pool: PagePool,
                 k: int = 4, plan_identity: bytes = None):
        if k < 1:
            raise ValueError("a speculative round needs at least one draft token")
        self.target, self.tpool = target, target_pool
        self.draft, self.dpool = draft, draft_pool
        self.k = k
        self.seqs: list[SpecSequence] = []
        # The 32-byte plan identity each completion record carries: the
        # caller's, or a digest of this round's shape.
        self.plan = plan_identity if plan_identity is not None else hashlib.sha256(
            f"ferric-amd greedy speculative round K={k}".encode()).digest()
        if len(self.plan) != 32:
            raise ValueError("plan identity must be 32 bytes")
        self.epoch = 0  # completion epoch: rounds settled so far

    def _run(self, runner, pool, rows, outputs):
        batch = pool.prepare(rows)
        out = runner.execute_batch(batch, outputs)
        pool.commit(batch)
        return out.choices

    def prefill(self, prompts):
        """Prefills every prompt into both models (one batch each); the
        target's greedy token after each prompt is the first anchor."""
        t_rows, d_rows, outs = [], [], []
        for p in prompts:
            ts, ds = self.tpool.admit(0), self.dpool.admit(0)
            self.seqs.append(SpecSequence(ts, ds, len(p), -1, emitted=[]))
            t_rows += [(ts, int(x)) for x in p]
            d_rows += [(ds, int(x)) for x in p]
            outs.append(len(t_rows) - 1)
        first = self._run(self.target, self.tpool, t_rows, outs)
        self._run(self.draft, self.dpool, d_rows, [])
        for s, tok in zip(self.seqs, first):
            s.anchor = int(tok)
            s.emitted.append(int(tok))
        return first

    def round(self) -> RoundStats:
        k, seqs = self.k, self.seqs
        # Draft catch-up: consume last round's final candidate where all were accepted.
        late = [s for s in seqs if s.catch_up >= 0]
        if late:
            self._run(self.draft, self.dpool, [(s.draft_sid, s.catch_up) for s in late], [])
            for s in late:
                s.catch_up = -1
        # K draft steps (decode batches of one row per sequence).
        draft = np.zeros((k, len(seqs)), dtype=np.uint32)  # iteration-major
        inputs = [s.anchor for s in seqs]
        for i in range(k):
            draft[i] = self._run(self.draft, self.dpool, [(s.draft_sid, int(t)) for s, t in zip(seqs, inputs)],
                                 list(range(len(seqs))))
            inputs = draft[i]
        # One target batch of K + 1 inputs per sequence, every row an output row.
        ids = token_assembly([s.anchor for s in seqs], draft, k)
        rows = [(s.target_sid, int(t)) for s, row in zip(seqs, ids) for t in row]
        batch = self.tpool.prepare(rows)
        choices = np.asarray(self.target.execute_batch(batch, list(range(len(rows)))).choices,
                             dtype=np.uint32).reshape(len(seqs), k + 1)
        accepted, emitted = [], []
        acc, ems = verify_greedy_batch(draft, choices)
        for j, s in enumerate(seqs):
            a = int(acc[j])
            em = [int(x) for x in ems[j, : a + 1]]
            c = s.cursor
            self.tpool.truncate(s.target_sid, c + a + 1)
            self.dpool.truncate(s.draft_sid, c + min(a + 1, k))
            if a == k:
                s.catch_up = int(draft[k - 1, j])
            s.cursor = c + a + 1
            s.anchor = em[-1]
            s.emitted += em
            accepted.append(a)
            emitted.append(em)
        # Completion records, built once both pools are settled (so a round
        # whose shape a record cannot hold still leaves every cursor in step).
        records = round_records(choices, draft, k, self.epoch, self.plan)
        self.epoch += 1
        return RoundStats(accepted, emitted, k, len(late), len(rows), records, draft, choices)
