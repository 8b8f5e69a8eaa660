"""Qwen3 tokenizer for the real-checkpoint path: byte-level BPE executed here.

The reference admits one exact tokenizer.json (crates/ferric-build/src/
fixtures/tokenizer/README.md: 11,422,654 bytes, SHA-256 aeb13307...) and runs
its own closed encode/decode program over it
(crates/ferric-build/src/tokenizer.rs parse/admission,
crates/ferric-build/src/tokenizer_execution.rs execution). This module does the
same, in its own code:

* admission (tokenizer.rs:330-546): the file's SHA-256, the closed schema
  (NFC normalizer; one Split pre-tokenizer with the Qwen3 expression, Isolated;
  ByteLevel without prefix space or regex; BPE without dropout, unknown token,
  byte fallback or affixes; ByteLevel decoder), the 151,643-entry base
  vocabulary and the 151,387 ordered merges, each checked against the
  reference's semantic digests (length-prefixed records, README.md), and the
  26 added tokens at IDs 151,643..151,668;
* encode (tokenizer_execution.rs:324-434): special added tokens rejected
  unless the policy allows them; the text split at added tokens (leftmost
  start, then the longest content, then the lowest ID); each plain span NFC
  normalized, split by the Qwen3 expression with unmatched gaps kept as
  pieces, and each piece's UTF-8 bytes mapped through the GPT-2 byte alphabet
  and merged by BPE (tokenizer_execution.rs:817-1200: repeatedly the
  lowest-ranked adjacent pair, the leftmost one on a rank tie, every
  non-overlapping occurrence of it in one pass);
* decode (tokenizer_execution.rs:1637-1800) to bytes, preserving added tokens
  or skipping the 14 special ones; unknown IDs are errors;
* the reference's bounds (tokenizer_execution.rs:19-118): 32 KiB input,
  128 KiB normalized text, 8,192 tokens, 128 KiB decoded bytes and a work
  budget. Work units follow the reference's charging points (one per scanned
  byte, normalized character, merged symbol and decoded byte; 1,024 per BPE
  pair lookup).

Unicode tables: NFC comes from the interpreter's `unicodedata` and the split
expression runs on the `regex` package. The reference uses Unicode 9.0.0 NFC
tables and Oniguruma's Unicode 16.0.0 tables; results can differ only for code
points assigned after those versions.
"""

from __future__ import annotations

import enum
import hashlib
import json
import struct
import unicodedata
from dataclasses import dataclass
from typing import Optional, Sequence

from .checkpoint import file_sha256

QWEN3_TOKENIZER_SHA256 = "aeb13307a71acd8fe81861d94ad54ab689df773318809eed3cbe794b4492dae4"
QWEN3_TOKENIZER_BYTES = 11_422_654
VOCABULARY_SEMANTIC_SHA256 = "d42824870d58ccbf38bc6d29b312cc4550c8543f448c45fe644dd041f3eff638"
MERGES_SEMANTIC_SHA256 = "1f8c784c660c1659a981d03c46deea0abcbf3fb4f6e85938e27281869890734f"
BASE_VOCABULARY_SIZE = 151_643
MERGE_COUNT = 151_387
ADDED_TOKEN_COUNT = 26
QWEN3_SPLIT_REGEX = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|"
                     r"\s*[\r\n]+|\s+(?!\S)|\s+")

MAX_INPUT_BYTES = 32 * 1024
MAX_NORMALIZED_BYTES = 128 * 1024
MAX_OUTPUT_TOKENS = 8192
MAX_OUTPUT_BYTES = 128 * 1024
MAX_WORK = 16 * 1024 * 1024
_PAIR_LOOKUP_WORK = (4 + 4) * 128  # charge_ordered_lookup(work, 4, 4)


class TokenizerError(ValueError):
    """Admission failure: the file is not the pinned Qwen3 tokenizer."""


class TokenizerExecutionError(ValueError):
    """A fail-closed encode/decode failure (TokenizerExecutionError,
    tokenizer_execution.rs:142-167). `kind` names the variant; `token_id`,
    `limit` and `actual` carry its fields where it has them."""

    def __init__(self, kind: str, message: str, **fields):
        super().__init__(message)
        self.kind = kind
        self.token_id = fields.get("token_id")
        self.limit = fields.get("limit")
        self.actual = fields.get("actual")


class SpecialTokenEncodePolicy(enum.Enum):
    REJECT = "reject"  # input holding any special added token fails
    ALLOW = "allow"    # special added tokens encode to their IDs


class SpecialTokenDecodePolicy(enum.Enum):
    PRESERVE = "preserve"  # every added token decodes to its content
    SKIP = "skip"          # the special added tokens decode to nothing


@dataclass(frozen=True)
class TokenizerLimits:
    """Caller bounds, each in 1..its hard ceiling (TokenizerExecutionLimits)."""

    input_bytes: int = MAX_INPUT_BYTES
    tokens: int = MAX_OUTPUT_TOKENS
    output_bytes: int = MAX_OUTPUT_BYTES
    work: int = MAX_WORK

    def validate(self) -> None:
        for value, ceiling in ((self.input_bytes, MAX_INPUT_BYTES), (self.tokens, MAX_OUTPUT_TOKENS),
                               (self.output_bytes, MAX_OUTPUT_BYTES), (self.work, MAX_WORK)):
            if not 0 < value <= ceiling:
                raise TokenizerExecutionError("InvalidLimits", "tokenizer execution limits are invalid")


def byte_level_alphabet() -> list:
    """The GPT-2 ByteLevel alphabet: byte b -> one code point. Printable
    Latin-1 bytes map to themselves, the other 68 bytes to 256, 257, ... in
    byte order."""
    keep = set(range(0x21, 0x7F)) | set(range(0xA1, 0xAD)) | set(range(0xAE, 0x100))
    out, extra = [], 0
    for b in range(256):
        if b in keep:
            out.append(chr(b))
        else:
            out.append(chr(256 + extra))
            extra += 1
    return out


def _field(h, data: bytes) -> None:
    h.update(struct.pack(">Q", len(data)))
    h.update(data)


class _Work:
    __slots__ = ("limit", "used")

    def __init__(self, limit: int):
        self.limit = limit
        self.used = 0

    def charge(self, amount: int) -> None:
        if amount > self.limit - self.used:
            raise TokenizerExecutionError("WorkLimit", f"tokenizer work exceeds limit {self.limit}", limit=self.limit)
        self.used += amount


def run_bpe(symbols: list, merge_ranks: dict):
    """BPE over symbol IDs (run_bpe, tokenizer_execution.rs:1117): while a
    ranked adjacent pair exists, take the lowest rank (the leftmost pair on a
    tie) and replace every non-overlapping occurrence of that pair, left to
    right, with its result. merge_ranks: (left, right) -> (rank, result).
    Returns (symbols, work units the reference charges for it)."""
    cost = 0
    while len(symbols) > 1:
        cost += (len(symbols) - 1) * _PAIR_LOOKUP_WORK
        best = None
        for i in range(len(symbols) - 1):
            rule = merge_ranks.get((symbols[i], symbols[i + 1]))
            if rule is not None and (best is None or rule[0] < best[0]):
                best = (rule[0], symbols[i], symbols[i + 1], rule[1])
        if best is None:
            break
        _, left, right, result = best
        merged = []
        i, n = 0, len(symbols)
        while i < n:
            cost += 1
            if i + 1 < n and symbols[i] == left and symbols[i + 1] == right:
                merged.append(result)
                i += 2
            else:
                merged.append(symbols[i])
                i += 1
        symbols = merged
    return list(symbols), cost


def reject_forbidden_special(data: bytes, added: list, work: _Work) -> None:
    """SpecialTokenForbidden for the first position (then the lowest ID)
    where a special added token's content occurs (tokenizer_execution.rs:491).
    added: [(content bytes, special, id)]."""
    for start in range(len(data)):
        work.charge(1)
        if data[start] != 0x3C:
            continue
        for content, special, tid in added:
            if not special:
                continue
            work.charge(len(content))
            if data.startswith(content, start):
                raise TokenizerExecutionError("SpecialTokenForbidden", f"special tokenizer token ID {tid} is "
                                              "forbidden", token_id=tid)


def find_added_token(data: bytes, cursor: int, added: list, work: _Work):
    """The leftmost added-token match at or after `cursor`: the longest
    content there, then the first in `added` order (tokenizer_execution.rs:582).
    Every content starts with '<'. Returns (start, content, special, id) or None."""
    for start in range(cursor, len(data)):
        work.charge(1)
        if data[start] != 0x3C:
            continue
        best = None
        for content, special, tid in added:
            work.charge(len(content))
            if data.startswith(content, start) and (best is None or len(content) > len(best[0])):
                best = (content, special, tid)
        if best is not None:
            return (start,) + best
    return None


def decode_bytes(ids: Sequence[int], vocab_bytes: list, added: list,
                 special_tokens: SpecialTokenDecodePolicy, limits: TokenizerLimits) -> bytes:
    """decode_to_bytes (tokenizer_execution.rs:1637): base IDs below
    BASE_VOCABULARY_SIZE decode through vocab_bytes, the next len(added) IDs
    to their content (nothing for a special one under SKIP); any other ID,
    or a base ID without bytes, is UnknownTokenId."""
    limits.validate()
    if len(ids) > limits.tokens:
        raise TokenizerExecutionError("TokenLimit", f"token count is {len(ids)}, limit is {limits.tokens}",
                                      limit=limits.tokens, actual=len(ids))
    work = _Work(limits.work)
    out = bytearray()
    for t in ids:
        work.charge(1)
        t = int(t)
        if 0 <= t < BASE_VOCABULARY_SIZE and t < len(vocab_bytes):
            piece = vocab_bytes[t]
        elif 0 <= t - BASE_VOCABULARY_SIZE < len(added) and added[t - BASE_VOCABULARY_SIZE][2] == t:
            content, special, _ = added[t - BASE_VOCABULARY_SIZE]
            piece = b"" if special and special_tokens == SpecialTokenDecodePolicy.SKIP else content
        else:
            raise TokenizerExecutionError("UnknownTokenId", f"unknown tokenizer token ID {t}", token_id=t)
        work.charge(len(piece))
        if len(out) + len(piece) > limits.output_bytes:
            raise TokenizerExecutionError("OutputByteLimit", f"decoded tokenizer bytes exceed limit "
                                          f"{limits.output_bytes}", limit=limits.output_bytes)
        out += piece
    return bytes(out)


class Qwen3Tokenizer:
    """Encode text to token IDs and decode IDs to bytes over the pinned
    Qwen3 tokenizer.json (AuthenticatedTokenizer)."""

    def __init__(self, path: str, sha256: Optional[str] = QWEN3_TOKENIZER_SHA256):
        if sha256 is not None:
            got = file_sha256(path)
            if got != sha256.lower():
                raise TokenizerError(f"{path}: SHA-256 {got}, expected {sha256}")
        with open(path, "rb") as f:
            doc = json.loads(f.read().decode("utf-8"))
        self._admit_schema(doc)
        vocab_ids = self._admit_vocabulary(doc["model"]["vocab"])
        merges = self._admit_merges(doc["model"]["merges"])
        self._admit_added(doc["added_tokens"])

        alphabet = byte_level_alphabet()
        to_byte = {c: b for b, c in enumerate(alphabet)}
        self._byte_token = [vocab_ids[c] for c in alphabet]
        self._vocab_bytes = []
        for token in self._tokens:
            try:
                self._vocab_bytes.append(bytes(to_byte[c] for c in token))
            except KeyError as e:
                raise TokenizerError(f"vocabulary symbol {e.args[0]!r} is outside ByteLevel") from None
        self._merge = {}
        for rank, (left, right) in enumerate(merges):
            try:
                key = (vocab_ids[left], vocab_ids[right])
                result = vocab_ids[left + right]
            except KeyError:
                raise TokenizerError(f"merge {rank} names a token outside the vocabulary") from None
            self._merge[key] = (rank, result)
        import regex  # the split expression needs Unicode property classes

        self._split = regex.compile(QWEN3_SPLIT_REGEX)
        self._piece_cache: dict = {}

    # ---- admission ----------------------------------------------------------
    @staticmethod
    def _admit_schema(doc: dict) -> None:
        def need(cond, where):
            if not cond:
                raise TokenizerError(f"unexpected tokenizer schema at {where}")

        need(doc.get("normalizer") == {"type": "NFC"}, "$.normalizer")
        pre = doc.get("pre_tokenizer") or {}
        steps = pre.get("pretokenizers") or []
        need(pre.get("type") == "Sequence" and len(steps) == 2, "$.pre_tokenizer")
        need(steps[0] == {"type": "Split", "pattern": {"Regex": QWEN3_SPLIT_REGEX}, "behavior": "Isolated",
                          "invert": False}, "$.pre_tokenizer.pretokenizers[0]")
        byte_level = {"type": "ByteLevel", "add_prefix_space": False, "trim_offsets": False, "use_regex": False}
        need(steps[1] == byte_level, "$.pre_tokenizer.pretokenizers[1]")
        need(doc.get("decoder") == byte_level, "$.decoder")
        model = doc.get("model") or {}
        need(model.get("type") == "BPE" and model.get("dropout") is None and model.get("unk_token") is None
             and model.get("continuing_subword_prefix") in ("", None) and model.get("end_of_word_suffix") in ("", None)
             and not model.get("fuse_unk") and not model.get("byte_fallback") and not model.get("ignore_merges"),
             "$.model")

    def _admit_vocabulary(self, vocab: dict) -> dict:
        if len(vocab) != BASE_VOCABULARY_SIZE:
            raise TokenizerError(f"base vocabulary has {len(vocab)} entries, expected {BASE_VOCABULARY_SIZE}")
        tokens = [None] * BASE_VOCABULARY_SIZE
        for token, i in vocab.items():
            if not isinstance(i, int) or not 0 <= i < BASE_VOCABULARY_SIZE or tokens[i] is not None:
                raise TokenizerError(f"vocabulary ID {i!r} of {token!r} is out of range or repeated")
            tokens[i] = token
        h = hashlib.sha256()
        _field(h, b"ferric.qwen3-tokenizer-vocab.v1")
        for i, token in enumerate(tokens):
            _field(h, struct.pack(">I", i))
            _field(h, token.encode("utf-8"))
        if h.hexdigest() != VOCABULARY_SEMANTIC_SHA256:
            raise TokenizerError("vocabulary semantic digest mismatch")
        self._tokens = tokens
        return dict(vocab)

    @staticmethod
    def _admit_merges(merges: list) -> list:
        if len(merges) != MERGE_COUNT:
            raise TokenizerError(f"{len(merges)} merges, expected {MERGE_COUNT}")
        h = hashlib.sha256()
        _field(h, b"ferric.qwen3-tokenizer-merges.v1")
        out = []
        for n, pair in enumerate(merges):
            if not (isinstance(pair, list) and len(pair) == 2 and all(isinstance(s, str) for s in pair)):
                raise TokenizerError(f"unexpected tokenizer schema at $.model.merges[{n}]")
            _field(h, struct.pack(">Q", n))
            _field(h, pair[0].encode("utf-8"))
            _field(h, pair[1].encode("utf-8"))
            out.append((pair[0], pair[1]))
        if h.hexdigest() != MERGES_SEMANTIC_SHA256:
            raise TokenizerError("merges semantic digest mismatch")
        return out

    def _admit_added(self, added: list) -> None:
        if len(added) != ADDED_TOKEN_COUNT:
            raise TokenizerError(f"{len(added)} added tokens, expected {ADDED_TOKEN_COUNT}")
        self._added = []  # (content bytes, special, id) in ID order
        for n, a in enumerate(added):
            want_id = BASE_VOCABULARY_SIZE + n
            if (a.get("id") != want_id or a.get("normalized") or a.get("single_word") or a.get("lstrip")
                    or a.get("rstrip") or not isinstance(a.get("content"), str) or not a["content"].startswith("<")):
                raise TokenizerError(f"unexpected tokenizer schema at $.added_tokens[{n}]")
            self._added.append((a["content"].encode("utf-8"), bool(a.get("special")), want_id))

    # ---- properties -----------------------------------------------------------
    @property
    def vocab_size(self) -> int:
        """Base vocabulary plus added tokens (151,669)."""
        return BASE_VOCABULARY_SIZE + len(self._added)

    @property
    def added_tokens(self) -> list:
        """[(content, special, id)] in ID order."""
        return [(c.decode("utf-8"), s, i) for c, s, i in self._added]

    # ---- encode ---------------------------------------------------------------
    def encode(self, text: str, special_tokens: SpecialTokenEncodePolicy = SpecialTokenEncodePolicy.REJECT,
               limits: TokenizerLimits = TokenizerLimits()) -> list:
        """Token IDs of `text` (no implicit special tokens)."""
        limits.validate()
        data = text.encode("utf-8")
        if len(data) > limits.input_bytes:
            raise TokenizerExecutionError("InputTooLarge", f"tokenizer input is {len(data)} bytes, limit is "
                                          f"{limits.input_bytes}", limit=limits.input_bytes, actual=len(data))
        work = _Work(limits.work)
        if special_tokens == SpecialTokenEncodePolicy.REJECT:
            reject_forbidden_special(data, self._added, work)
        out: list = []
        cursor = 0
        while cursor < len(data):
            found = find_added_token(data, cursor, self._added, work)
            end = found[0] if found else len(data)
            if end > cursor:
                self._encode_plain(data[cursor:end].decode("utf-8"), limits, work, out)
            if found is None:
                break
            start, content, special, tid = found
            if special and special_tokens == SpecialTokenEncodePolicy.REJECT:
                raise TokenizerExecutionError("SpecialTokenForbidden", f"special tokenizer token ID {tid} is "
                                              "forbidden", token_id=tid)
            self._push(out, tid, limits.tokens)
            cursor = start + len(content)
        return out

    def _encode_plain(self, text: str, limits: TokenizerLimits, work: _Work, out: list) -> None:
        normalized = unicodedata.normalize("NFC", text)
        work.charge(len(normalized))
        size = len(normalized.encode("utf-8"))
        if size > MAX_NORMALIZED_BYTES:
            size = 0
            for ch in normalized:
                size += len(ch.encode("utf-8"))
                if size > MAX_NORMALIZED_BYTES:
                    break
            raise TokenizerExecutionError("NormalizedInputTooLarge", f"normalized tokenizer input is {size} bytes, "
                                          f"limit is {MAX_NORMALIZED_BYTES}", limit=MAX_NORMALIZED_BYTES,
                                          actual=size)
        previous = 0
        for m in self._split.finditer(normalized):
            start, end = m.span()
            work.charge(end - previous)
            if start != previous:
                self._encode_piece(normalized[previous:start], limits, work, out)
            self._encode_piece(normalized[start:end], limits, work, out)
            previous = end
        if previous != len(normalized):
            work.charge(len(normalized) - previous)
            self._encode_piece(normalized[previous:], limits, work, out)

    def _encode_piece(self, piece: str, limits: TokenizerLimits, work: _Work, out: list) -> None:
        data = piece.encode("utf-8")
        work.charge(len(data))
        ids = self._piece_cache.get(data)
        if ids is None:
            ids, cost = run_bpe([self._byte_token[b] for b in data], self._merge)
            if len(self._piece_cache) < 65536:
                self._piece_cache[data] = (ids, cost)
        else:
            ids, cost = ids
        work.charge(cost)
        for t in ids:
            self._push(out, t, limits.tokens)

    @staticmethod
    def _push(out: list, token: int, limit: int) -> None:
        if len(out) + 1 > limit:
            raise TokenizerExecutionError("TokenLimit", f"token count is {len(out) + 1}, limit is {limit}",
                                          limit=limit, actual=len(out) + 1)
        out.append(token)

    # ---- decode ---------------------------------------------------------------
    def decode_to_bytes(self, ids: Sequence[int],
                        special_tokens: SpecialTokenDecodePolicy = SpecialTokenDecodePolicy.PRESERVE,
                        limits: TokenizerLimits = TokenizerLimits()) -> bytes:
        """The bytes of `ids` (an arbitrary slice of base tokens need not be
        valid UTF-8)."""
        return decode_bytes(ids, self._vocab_bytes, self._added, special_tokens, limits)

    def decode(self, ids: Sequence[int], skip_special: bool = False) -> str:
        """Text of `ids`; byte sequences that are not UTF-8 become U+FFFD."""
        policy = SpecialTokenDecodePolicy.SKIP if skip_special else SpecialTokenDecodePolicy.PRESERVE
        return self.decode_to_bytes(ids, policy).decode("utf-8", errors="replace")
