"""Qwen3 tokenizer (CPU): the reference's 640-case differential fixture
(crates/ferric-build/src/fixtures/tokenizer/qwen3-tokenizer-differential.txt,
committed under tests/golden as data) and the real-weight smoke KAT of
docs/M1_QWEN3_TP_ENGINEERING.md:80-82 (a five-token prompt, generated ids
[12095, 13] decoding to " Paris."). The tokenizer.json itself (11 MB) is
read from FERRIC_QWEN3_TOKENIZER or the reference checkout when present."""

import os
from pathlib import Path

import pytest

from ferric_amd.tokenizer import QWEN3_TOKENIZER_SHA256, Qwen3Tokenizer, TokenizerError

GOLDEN = Path(__file__).parent / "golden" / "qwen3_tokenizer_differential.txt"
CANDIDATES = [os.environ.get("FERRIC_QWEN3_TOKENIZER", ""),
              "/root/reference/crates/ferric-build/src/fixtures/tokenizer/qwen3-tokenizer.json"]
PATH = next((p for p in CANDIDATES if p and os.path.exists(p)), None)
needs_file = pytest.mark.skipif(PATH is None, reason="Qwen3 tokenizer.json not available")


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
def test_differential_fixture():
    tok = Qwen3Tokenizer(PATH)
    bad = [(t, e, tok.encode(t)) for t, e in cases() if tok.encode(t) != e]
    assert not bad, bad[:3]


@needs_file
def test_paris_known_answer():
    tok = Qwen3Tokenizer(PATH)
    assert tok.decode([12095, 13]) == " Paris."
    assert len(tok.encode("The capital of France is")) == 5
    assert tok.vocab_size == 151669


def test_pin_mismatch(tmp_path):
    p = tmp_path / "tokenizer.json"
    p.write_text("{}")
    with pytest.raises(TokenizerError, match="SHA-256"):
        Qwen3Tokenizer(str(p))
