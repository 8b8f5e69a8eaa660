"""Qwen3 tokenizer for the real-checkpoint path.

The reference admits one exact tokenizer.json (crates/ferric-build/src/
fixtures/tokenizer/README.md: 11,422,654 bytes, SHA-256 aeb13307...) and
executes its byte-level BPE natively (crates/ferric-build/src/
tokenizer_execution.rs). Here the same file is executed by the Hugging Face
`tokenizers` library, the implementation the reference's own 640-case
differential fixture was generated with (tokenizers 0.22.2). Encoding adds no
special tokens, as the reference's prompt path does.
"""

from __future__ import annotations

from typing import Optional, Sequence

from .checkpoint import file_sha256

QWEN3_TOKENIZER_SHA256 = "aeb13307a71acd8fe81861d94ad54ab689df773318809eed3cbe794b4492dae4"


class TokenizerError(ValueError):
    pass


class Qwen3Tokenizer:
    """encode(text) -> ids and decode(ids) -> text over a Qwen3 tokenizer.json."""

    def __init__(self, path: str, sha256: Optional[str] = QWEN3_TOKENIZER_SHA256):
        if sha256 is not None:
            got = file_sha256(path)
            if got != sha256.lower():
                raise TokenizerError(f"{path}: SHA-256 {got}, expected {sha256}")
        try:
            from tokenizers import Tokenizer
        except ImportError as e:  # pragma: no cover - the image ships it
            raise TokenizerError("the `tokenizers` package is required for the real-checkpoint path") from e
        self._tok = Tokenizer.from_file(str(path))

    @property
    def vocab_size(self) -> int:
        return self._tok.get_vocab_size(with_added_tokens=True)

    def encode(self, text: str) -> list:
        return list(self._tok.encode(text, add_special_tokens=False).ids)

    def decode(self, ids: Sequence[int]) -> str:
        return self._tok.decode([int(i) for i in ids], skip_special_tokens=False)
