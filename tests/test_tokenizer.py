"""Qwen3 tokenizer (CPU).

Pins for ferric_amd/tokenizer.py:
* the reference's 640-case differential fixture
  (crates/ferric-build/src/fixtures/tokenizer/qwen3-tokenizer-differential.txt,
  committed under tests/golden as data), encoded with special tokens allowed;
* the reference's own known-answer vectors and policy cases
  (crates/ferric-build/src/tokenizer_execution.rs:1848-2276: encode and decode
  fixtures, added/special policies, BPE rank ties, added-token overlap,
  decode holes, every bound) restated as data;
* a seeded differential run against the `tokenizers` 0.22.2 package (the
  implementation the fixture was generated with) over random strings built
  from the inputs the expression and NFC treat differently;
* the real-weight smoke KAT of docs/M1_QWEN3_TP_ENGINEERING.md:80-82 (a
  five-token prompt, generated ids [12095, 13] decoding to " Paris.").
The tokenizer.json itself (11 MB) is read from FERRIC_QWEN3_TOKENIZER or the
reference checkout when present."""

import json
import os
import random
from pathlib import Path

import pytest

from ferric_amd import tokenizer as tk
from ferric_amd.tokenizer import (QWEN3_TOKENIZER_SHA256, Qwen3Tokenizer, SpecialTokenDecodePolicy as D,
                                  SpecialTokenEncodePolicy as E, TokenizerError, TokenizerExecutionError,
                                  TokenizerLimits)

GOLDEN = Path(__file__).parent / "golden" / "qwen3_tokenizer_differential.txt"
CANDIDATES = [os.environ.get("FERRIC_QWEN3_TOKENIZER", ""),
              "/root/reference/crates/ferric-build/src/fixtures/tokenizer/qwen3-tokenizer.json"]
PATH = next((p for p in CANDIDATES if p and os.path.exists(p)), None)
needs_file = pytest.mark.skipif(PATH is None, reason="Qwen3 tokenizer.json not available")


@pytest.fixture(scope="module")
def tok():
    return Qwen3Tokenizer(PATH)


def cases():
    for line in GOLDEN.read_text().splitlines():
        if line.startswith("#"):
            continue
        text_hex, ids = line.split("\t")
        text = "" if text_hex == "-" else bytes.fromhex(text_hex).decode("utf-8")
        yield text, [] if ids == "-" else [int(x) for x in ids.split(",")]


def test_fixture_header_pins_the_tokenizer():
    head = [l for l in GOLDEN.read_text().splitlines() if l.startswith("#")]
    assert f"# tokenizer-sha256={QWEN3_TOKENIZER_SHA256}" in head
    assert sum(1 for _ in cases()) == 640


@needs_file
def test_differential_fixture(tok):
    bad = [(t, e, tok.encode(t, E.ALLOW)) for t, e in cases() if tok.encode(t, E.ALLOW) != e]
    assert not bad, bad[:3]


# tokenizer_execution.rs:1848-1886 (encoded under the Reject policy)
ENCODE_KATS = [
    ("", []),
    ("hello", [14990]),
    ("Hello world", [9707, 1879]),
    ("hello   world", [14990, 256, 1879]),
    ("I'm testing!", [40, 2776, 7497, 0]),
    ("1 23\nnext", [16, 220, 17, 18, 198, 3600]),
    ("tabs\twork", [30993, 97038]),
    ("line\r\nend", [1056, 319, 408]),
    (" punctuation!?", [61503, 57390]),
    ("A.B", [32, 1785]),
    ("trailing   ", [376, 14277, 262]),
    ("I'RE", [40, 94153]),
    ("\0\x7f", [188, 221]),
    ("e\u0301", [963]),
    ("\u00e9", [963]),
    ("\u4e2d\u6587", [104811]),
    ("\u0661\u0662", [149, 94, 149, 95]),
]

# tokenizer_execution.rs:1890-1912 (decoded under Preserve)
DECODE_KATS = [
    ([14990], b"hello"),
    ([9707, 1879], b"Hello world"),
    ([40, 2776, 7497, 0], b"I'm testing!"),
    ([16, 220, 17, 18, 198, 3600], b"1 23\nnext"),
    ([30993, 97038], b"tabs\twork"),
    ([1056, 319, 408], b"line\r\nend"),
    ([188, 222, 187], bytes([0, 128, 255])),
]


@needs_file
def test_reference_encode_and_decode_known_answers(tok):
    for text, ids in ENCODE_KATS:
        assert tok.encode(text, E.REJECT) == ids, text
        assert tok.encode(text, E.REJECT) == ids, text  # deterministic on repeat
    for ids, data in DECODE_KATS:
        assert tok.decode_to_bytes(ids, D.PRESERVE) == data


@needs_file
def test_added_and_special_token_policy(tok):
    # tokenizer_execution.rs:1915-2027
    assert tok.encode("<think>ok</think>", E.REJECT) == [151667, 562, 151668]
    with pytest.raises(TokenizerExecutionError) as e:
        tok.encode("<|im_start|>user\nHello<|im_end|>", E.REJECT)
    assert (e.value.kind, e.value.token_id) == ("SpecialTokenForbidden", 151644)
    with pytest.raises(TokenizerExecutionError) as e:
        tok.encode("é prefix <|im_end|>", E.REJECT)
    assert (e.value.kind, e.value.token_id) == ("SpecialTokenForbidden", 151645)
    ids = tok.encode("<|im_start|>user\nHello<|im_end|>", E.ALLOW)
    assert ids == [151644, 872, 198, 9707, 151645]
    assert tok.decode_to_bytes(ids, D.PRESERVE) == b"<|im_start|>user\nHello<|im_end|>"
    assert tok.decode_to_bytes(ids, D.SKIP) == b"user\nHello"

    added = tok.added_tokens
    assert len(added) == 26 and sum(s for _, s, _ in added) == 14
    assert all(s for _, s, _ in added[:14]) and not any(s for _, s, _ in added[14:])
    for content, special, tid in added:
        assert tid == 151643 + added.index((content, special, tid))
        if special:
            with pytest.raises(TokenizerExecutionError) as e:
                tok.encode(content, E.REJECT)
            assert e.value.token_id == tid
        else:
            assert tok.encode(content, E.REJECT) == [tid]
        assert tok.encode(content, E.ALLOW) == [tid]
        assert tok.decode_to_bytes([tid], D.PRESERVE) == content.encode()
        assert tok.decode_to_bytes([tid], D.SKIP) == (b"" if special else content.encode())


def test_byte_level_alphabet_is_a_bijection():
    alphabet = tk.byte_level_alphabet()
    assert len(set(alphabet)) == 256
    assert alphabet[ord("A")] == "A" and alphabet[0x20] == "Ġ" and alphabet[0x0A] == "Ċ"
    assert "€" not in alphabet


def test_bpe_rank_ties_and_simultaneous_merges():
    # tokenizer_execution.rs:2077-2111
    assert tk.run_bpe([1, 2, 3], {(1, 2): (10, 4), (2, 3): (1, 5)})[0] == [1, 5]  # lower rank first
    assert tk.run_bpe([1, 2, 3], {(1, 2): (1, 4), (2, 3): (1, 5)})[0] == [4, 3]  # rank tie: earliest pair
    assert tk.run_bpe([1, 2, 1, 2, 1], {(1, 2): (0, 9)})[0] == [9, 9, 1]       # every non-overlapping pair
    assert tk.run_bpe([7, 7, 7], {(7, 7): (0, 8)})[0] == [8, 7]                # overlapping run, left to right
    work = tk._Work(1)
    with pytest.raises(TokenizerExecutionError) as e:
        work.charge(tk.run_bpe([1, 2], {(1, 2): (0, 9)})[1])
    assert (e.value.kind, e.value.limit, work.used) == ("WorkLimit", 1, 0)


def test_added_token_overlap_uses_earliest_longest_lowest():
    # tokenizer_execution.rs:2114-2156
    added = [(b"<ab", False, 10), (b"<abc", False, 11), (b"<abc", False, 12), (b"<z", True, 13)]
    data = b"x<abc<z"
    start, content, special, tid = tk.find_added_token(data, 0, added, tk._Work(tk.MAX_WORK))
    assert (start, tid) == (1, 11)
    start, content, special, tid = tk.find_added_token(data, 2, added, tk._Work(tk.MAX_WORK))
    assert (start, tid) == (5, 13)
    with pytest.raises(TokenizerExecutionError) as e:
        tk.reject_forbidden_special(data, added, tk._Work(tk.MAX_WORK))
    assert e.value.token_id == 13


def test_decode_preserves_bytes_skips_only_special_and_rejects_holes():
    # tokenizer_execution.rs:2159-2205
    base = tk.BASE_VOCABULARY_SIZE
    vocab = [bytes([0, 0xFF])]
    added = [(b"<s>", True, base), (b"plain", False, base + 1)]
    limits = TokenizerLimits(1, 4, 32, 1024)
    ids = [0, base, base + 1]
    assert tk.decode_bytes(ids, vocab, added, D.PRESERVE, limits) == b"\0\xff<s>plain"
    assert tk.decode_bytes(ids, vocab, added, D.SKIP, limits) == b"\0\xffplain"
    for hole in (1, base + 2):
        with pytest.raises(TokenizerExecutionError) as e:
            tk.decode_bytes([hole], vocab, added, D.PRESERVE, limits)
        assert (e.value.kind, e.value.token_id) == ("UnknownTokenId", hole)


@needs_file
def test_every_bound_fails_closed(tok):
    # tokenizer_execution.rs:2208-2275
    def err(fn):
        with pytest.raises(TokenizerExecutionError) as e:
            fn()
        return e.value

    e = err(lambda: tok.encode("hello", E.REJECT, TokenizerLimits(4, 8, 8, 1024)))
    assert (e.kind, e.limit, e.actual) == ("InputTooLarge", 4, 5)
    e = err(lambda: tok.encode("hello world", E.REJECT, TokenizerLimits(32, 1, 32, tk.MAX_WORK)))
    assert (e.kind, e.limit, e.actual) == ("TokenLimit", 1, 2)
    e = err(lambda: tok.encode("hello", E.REJECT, TokenizerLimits(32, 8, 32, 1)))
    assert (e.kind, e.limit) == ("WorkLimit", 1)
    e = err(lambda: tok.decode_to_bytes([14990], D.PRESERVE, TokenizerLimits(32, 8, 4, 1024)))
    assert (e.kind, e.limit) == ("OutputByteLimit", 4)
    e = err(lambda: tok.decode_to_bytes([151669], D.PRESERVE))
    assert (e.kind, e.token_id) == ("UnknownTokenId", 151669)
    e = err(lambda: tok.encode("x", E.REJECT, TokenizerLimits(tk.MAX_INPUT_BYTES + 1, 1, 1, 1)))
    assert e.kind == "InvalidLimits"
    e = err(lambda: tok.decode_to_bytes([1] * 9, D.PRESERVE, TokenizerLimits(32, 8, 32, 1024)))
    assert (e.kind, e.limit, e.actual) == ("TokenLimit", 8, 9)


# Pools the random strings draw from: each stresses a branch of the split
# expression, NFC or the added-token scan.
POOLS = [
    list("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ"),
    list("0123456789") + ["١", "٢", "²", "Ⅳ", "１"],
    list("!?.,;:'\"()[]{}<>|/\\-_=+*&^%$#@~`"),
    [" ", "  ", "\t", "\n", "\r", "\r\n", "\x0b", "\x0c", "\x85", "\xa0", " ", "　", "\x1c", "\x1f"],
    ["'s", "'S", "'t", "'re", "'RE", "'ve", "'m", "'ll", "'LL", "'d", "'D", "'x"],
    ["中", "文", "日本", "한", "\u1100\u1161", "कि", "שלום",
     "ال", "\u00e9", "e\u0301", "A\u030a", "\u212b", "\u1e9b\u0323", "ß", "İ", "Σ"],
    ["\U0001f600", "\U0001f44d\U0001f3fd", "❤️", "\U0001d400", "‍", "﻿", "\x00", "\x7f"],
    ["<|im_start|>", "<|im_end|>", "<|endoftext|>", "<think>", "</think>", "<tool_call>", "<|im_", "<|", "<",
     "<|vision_start|><|image_pad|>", "<think"],
]


@needs_file
def test_random_strings_match_the_tokenizers_package(tok):
    tokenizers = pytest.importorskip("tokenizers")
    hf = tokenizers.Tokenizer.from_file(PATH)
    rng = random.Random(20261202)
    bad = []
    for n in range(3000):
        parts = []
        for _ in range(rng.randint(1, 24)):
            pool = POOLS[rng.randrange(len(POOLS))]
            parts.append(pool[rng.randrange(len(pool))])
        text = "".join(parts)
        want = hf.encode(text, add_special_tokens=False).ids
        got = tok.encode(text, E.ALLOW)
        if got != want:
            bad.append((text, want, got))
            continue
        assert tok.decode_to_bytes(got, D.PRESERVE) == hf.decode(got, skip_special_tokens=False).encode()
    assert not bad, bad[:3]


@needs_file
def test_paris_known_answer(tok):
    assert tok.decode([12095, 13]) == " Paris."
    assert len(tok.encode("The capital of France is")) == 5
    assert tok.vocab_size == 151669


def test_pin_mismatch(tmp_path):
    p = tmp_path / "tokenizer.json"
    p.write_text("{}")
    with pytest.raises(TokenizerError, match="SHA-256"):
        Qwen3Tokenizer(str(p))


def test_schema_and_vocabulary_admission(tmp_path):
    # Unpinned files still go through the closed schema and the semantic digests.
    byte_level = {"type": "ByteLevel", "add_prefix_space": False, "trim_offsets": False, "use_regex": False}
    doc = {"added_tokens": [], "normalizer": {"type": "NFC"},
           "pre_tokenizer": {"type": "Sequence", "pretokenizers": [
               {"type": "Split", "pattern": {"Regex": tk.QWEN3_SPLIT_REGEX}, "behavior": "Isolated",
                "invert": False}, byte_level]},
           "decoder": byte_level,
           "model": {"type": "BPE", "dropout": None, "unk_token": None, "continuing_subword_prefix": "",
                     "end_of_word_suffix": "", "fuse_unk": False, "byte_fallback": False, "ignore_merges": False,
                     "vocab": {"a": 0}, "merges": []}}
    p = tmp_path / "t.json"
    p.write_text(json.dumps(doc))
    with pytest.raises(TokenizerError, match="base vocabulary has 1 entries"):
        Qwen3Tokenizer(str(p), sha256=None)
    doc["normalizer"] = {"type": "NFKC"}
    p.write_text(json.dumps(doc))
    with pytest.raises(TokenizerError, match=r"\$\.normalizer"):
        Qwen3Tokenizer(str(p), sha256=None)
