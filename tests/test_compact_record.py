"""Compact completion records (ferric_qwen3_compact_completion_v1,
device/qwen3-all-kernels-v1/src/logits.rs:279) on any host: the oracle's
restatement and the library's fh_compact_completion against the reference's
byte-exact vectors and read traces (device/qwen3-logits-v1/tests/reference.rs:
289-431, 433-608, 610-614)."""

import ctypes
import struct

import numpy as np
import pytest

import ferric_amd
from oracle import oracle as orc

VOCAB = 151936
INVALID = VOCAB


def token(record, i):
    return struct.unpack_from("<I", record, 52 + 4 * i)[0]


def lib_records(choices, draft, lives, slots, generations, epochs, plans, sequences, active_tokens, k):
    """fh_compact_completion over every sequence; None where it refuses."""
    lib = ferric_amd.load()
    u32 = lambda a: np.ascontiguousarray(np.asarray(a, np.uint32).reshape(-1))  # noqa: E731
    c, d = u32(choices), u32(draft if k else [0])
    lv, sl, gn = u32(lives), u32(slots), u32(generations)
    ep = np.ascontiguousarray(np.asarray(epochs, np.uint64))
    pl = np.frombuffer(b"".join(bytes(p) for p in plans), np.uint8).copy()
    out = np.full(sequences * 120, 0xEE, np.uint8)
    p32 = ctypes.POINTER(ctypes.c_uint32)
    p8 = ctypes.POINTER(ctypes.c_uint8)
    st = lib.fh_compact_completion(c.ctypes.data_as(p32), d.ctypes.data_as(p32) if k else None,
                                   lv.ctypes.data_as(p32), sl.ctypes.data_as(p32), gn.ctypes.data_as(p32),
                                   ep.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)), pl.ctypes.data_as(p8),
                                   sequences, active_tokens, k, out.ctypes.data_as(p8))
    if st != 0:
        assert np.all(out == 0xEE), "nothing is written when a sequence is refused"
        return None
    return [bytes(out[i * 120:(i + 1) * 120]) for i in range(sequences)]


def both(choices, draft, live, slot, generation, epoch, plan, sequences, sequence, active_tokens, k):
    """The oracle's record and trace for one sequence, checked against the
    library on a one-live-sequence batch of the same geometry."""
    rec, trace = orc.compact_record(choices, draft, live, slot, generation, epoch, plan, sequences, sequence,
                                    active_tokens, k)
    lives = [live if s == sequence else 0 for s in range(sequences)]
    got = lib_records(choices, draft, lives, [slot] * sequences, [generation] * sequences, [epoch] * sequences,
                      [plan] * sequences, sequences, active_tokens, k)
    if rec is None:
        assert got is None
    else:
        assert got is not None and got[sequence] == rec
        assert all(r == bytes(120) for s, r in enumerate(got) if s != sequence)
    return rec, trace


def test_direct_record_uses_final_live_row_and_never_needs_draft_data():
    plan = bytearray(32)
    plan[0], plan[31] = 0x44, 0x88
    choices = [0] * 128
    choices[:3] = [17, 23, 29]
    rec, trace = both(choices, [], 3, 7, 9, 0x1122334455667788, plan, 1, 0, 128, 0)
    assert rec[0:4] == struct.pack("<I", 7)
    assert rec[4:8] == struct.pack("<I", 9)
    assert rec[8:16] == struct.pack("<Q", 0x1122334455667788)
    assert rec[16:48] == bytes(plan)
    assert rec[48] == 0 and rec[49] == 1 and rec[50:52] == b"\0\0"
    assert token(rec, 0) == 29
    assert rec[56:] == bytes(64)
    assert trace == [("choice", 2)]


def test_speculative_record_emits_accepted_prefix_then_correction_or_bonus():
    plan = bytes([0x5A]) * 32
    mismatch, _ = both([10, 20, 30, 40, 50], [10, 20, 77, 88], 5, 1, 2, 3, plan, 1, 0, 5, 4)
    assert mismatch[48:52] == bytes([2, 3, 0, 0])
    assert [token(mismatch, i) for i in range(3)] == [10, 20, 30]
    assert mismatch[64:] == bytes(56)
    bonus, trace = both([10, 20, 30, 40, 99], [10, 20, 30, 40], 5, 1, 2, 3, plan, 1, 0, 5, 4)
    assert bonus[48:52] == bytes([4, 5, 0, 0])
    assert [token(bonus, i) for i in range(5)] == [10, 20, 30, 40, 99]
    assert bonus[72:] == bytes(48)
    assert trace == [("draft", 0), ("choice", 0), ("draft", 1), ("choice", 1), ("draft", 2), ("choice", 2),
                     ("draft", 3), ("choice", 3), ("choice", 4)]


def test_speculative_prefix_boundaries_are_byte_exact():
    plan = bytes([0x5A]) * 32
    choices = [10, 20, 30, 40, 99]
    for draft, accepted in [([77, 88, 89, 90], 0), ([10, 20, 77, 90], 2), ([10, 20, 30, 77], 3),
                            ([10, 20, 30, 40], 4)]:
        rec, _ = both(choices, draft, 5, 1, 2, 3, plan, 1, 0, 5, 4)
        assert rec[0:4] == struct.pack("<I", 1) and rec[4:8] == struct.pack("<I", 2)
        assert rec[8:16] == struct.pack("<Q", 3) and rec[16:48] == plan
        assert rec[48:52] == bytes([accepted, accepted + 1, 0, 0])
        for i in range(accepted):
            assert token(rec, i) == draft[i]
        assert token(rec, accepted) == choices[accepted]
        assert rec[52 + (accepted + 1) * 4:] == bytes(120 - 52 - (accepted + 1) * 4)


def test_mismatch_stops_later_validation_and_reads():
    rec, trace = both([10, 20, INVALID, 40, 99], [10, 77, INVALID, INVALID], 5, 1, 2, 3, bytes([0x5A]) * 32, 1, 0,
                      5, 4)
    assert rec is not None
    assert rec[48:52] == bytes([1, 2, 0, 0])
    assert token(rec, 0) == 10 and token(rec, 1) == 20
    assert rec[60:] == bytes(60)
    assert trace == [("draft", 0), ("choice", 0), ("draft", 1), ("choice", 1), ("choice", 1)]


def test_invalid_tokens_before_or_at_mismatch_are_rejected_after_the_pair_reads():
    for choices, draft in [([10, INVALID, 30, 40, 99], [10, 20, 77, 88]),
                           ([10, 20, 30, 40, 99], [10, INVALID, 77, 88])]:
        rec, trace = both(choices, draft, 5, 1, 2, 3, bytes([0x5A]) * 32, 1, 0, 5, 4)
        assert rec is None
        assert trace == [("draft", 0), ("choice", 0), ("draft", 1), ("choice", 1)]


@pytest.mark.parametrize("sequences,active_tokens,k", [(1, 1, 0), (1, 128, 0), (1, 512, 0), (1, 2048, 0),
                                                       (8, 1, 0), (8, 128, 0), (32, 1, 0), (1, 5, 4), (8, 5, 4),
                                                       (1, 9, 8), (1, 17, 16), (32, 5, 4)])
def test_accepted_bound_for_every_admitted_profile(sequences, active_tokens, k):
    # The reference's admitted profiles (reference.rs:482-608), plus the
    # 32-sequence K = 4 round of the speculative workload, all sequences at once.
    choices = np.arange(100, 100 + sequences * active_tokens, dtype=np.uint32)
    plan = bytes([0x5A]) * 32
    n = sequences
    if k == 0:
        got = lib_records(choices, [], [active_tokens] * n, [1] * n, [2] * n, [3] * n, [plan] * n, n,
                          active_tokens, 0)
        for s in range(n):
            rec, trace = orc.compact_record(choices, [], active_tokens, 1, 2, 3, plan, n, s, active_tokens, 0)
            ci = s * active_tokens + active_tokens - 1
            assert rec == got[s] and rec[48] == 0 and rec[49] == 1 and token(rec, 0) == choices[ci]
            assert trace == [("choice", ci)]
        return
    all_match = np.array([[choices[s * active_tokens + c] for s in range(n)] for c in range(k)], np.uint32)
    mismatch_at = k // 2
    mismatch = all_match.copy()
    for s in range(n):
        mismatch[mismatch_at, s] = choices[s * active_tokens + mismatch_at] + 1
    for draft, expected in [(all_match, k), (mismatch, mismatch_at)]:
        got = lib_records(choices, draft, [active_tokens] * n, [1] * n, [2] * n, [3] * n, [plan] * n, n,
                          active_tokens, k)
        for s in range(n):
            rec, trace = orc.compact_record(choices, draft, active_tokens, 1, 2, 3, plan, n, s, active_tokens, k)
            assert rec == got[s]
            assert rec[48] == expected and rec[49] == expected + 1 and rec[49] <= 17
            for c in range(expected):
                assert token(rec, c) == draft[c, s]
            ci = s * active_tokens + expected
            assert token(rec, expected) == choices[ci]
            compared = k if expected == k else expected + 1
            want = []
            for c in range(compared):
                want += [("draft", c * n + s), ("choice", s * active_tokens + c)]
            assert trace == want + [("choice", ci)]


def test_inactive_record_is_all_zero_without_request_authority():
    rec, trace = both([0], [], 0, 0xFFFFFFFF, 0, 0, bytes(32), 1, 0, 1, 0)
    assert rec == bytes(120) and trace == []


@pytest.mark.parametrize("field", ["slot", "generation", "plan", "live", "spec_live"])
def test_request_authority_rejections(field):
    # The kernel traps on slot >= 32, generation 0, an all-zero plan identity,
    # live > active_tokens and (speculative) a partial live width
    # (logits.rs:326-366); the library refuses the batch and writes nothing.
    plan = bytes([1]) + bytes(31)
    args = dict(choices=[10, 20, 30, 40, 99], draft=[10, 20, 30, 40], live=5, slot=31, generation=1, epoch=0,
                plan=plan, sequences=1, sequence=0, active_tokens=5, k=4)
    assert both(**args)[0] is not None
    bad = {"slot": dict(slot=32), "generation": dict(generation=0), "plan": dict(plan=bytes(32)),
           "live": dict(live=6), "spec_live": dict(live=3)}[field]
    assert both(**dict(args, **bad))[0] is None


def test_geometry_rejections():
    plan = [bytes([7]) * 32]
    ok = dict(choices=[1, 2, 3, 4, 5], draft=[1, 2, 3, 4], lives=[5], slots=[0], generations=[1], epochs=[0],
              plans=plan, sequences=1, active_tokens=5, k=4)
    assert lib_records(**ok) is not None
    assert lib_records(**dict(ok, active_tokens=4)) is None      # active_tokens != K + 1
    assert lib_records(**dict(ok, k=17, active_tokens=18)) is None  # K beyond 16
    many = dict(choices=[1] * 33, draft=[], lives=[1] * 33, slots=[0] * 33, generations=[1] * 33,
                epochs=[0] * 33, plans=plan * 33, sequences=33, active_tokens=1, k=0)
    assert lib_records(**many) is None                            # more sequences than the grid bound
