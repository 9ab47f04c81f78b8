"""Text in and out of the engine (liteinfer/tokenizer.py), over a local tokenizer file.

The reference wraps Hugging Face's `AutoTokenizer.from_pretrained(dir,
local_files_only=True)`; no checkpoint exists here, so `make_wordlevel`
writes a word-level `tokenizer.json` whose vocabulary is ``tok0`` ..
``tok{V-1}`` (token id i is the word ``tok{i}``, words split on whitespace)
and `Tokenizer` loads any such local file with the `tokenizers` library.
Random token ids rendered this way round-trip exactly, which is what the
end-to-end configuration's synthetic prompts need.
"""

from __future__ import annotations

from pathlib import Path

from tokenizers import Tokenizer as _HfTokenizer
from tokenizers import models, pre_tokenizers

TOKENIZER_FILE = "tokenizer.json"


def make_wordlevel(vocab_size: int, model_dir: str | Path) -> Path:
    """Write a word-level tokenizer of `vocab_size` words ``tok<i>`` into `model_dir`; returns its file."""
    if vocab_size < 1:
        raise ValueError("vocab_size must be >= 1")
    tok = _HfTokenizer(models.WordLevel({f"tok{i}": i for i in range(vocab_size)}, unk_token=None))
    tok.pre_tokenizer = pre_tokenizers.WhitespaceSplit()
    path = Path(model_dir) / TOKENIZER_FILE
    path.parent.mkdir(parents=True, exist_ok=True)
    tok.save(str(path))
    return path


class Tokenizer:
    """encode / decode / vocab_size / eos_token_ids, as liteinfer's `Tokenizer` (tokenizer.py:21-50)."""

    def __init__(self, model_dir: str | Path) -> None:
        path = Path(model_dir) / TOKENIZER_FILE
        if not path.is_file():
            raise FileNotFoundError(f"no {TOKENIZER_FILE} in {model_dir} (only local tokenizer files are read)")
        self._tok = _HfTokenizer.from_file(str(path))
        # A word-level vocabulary of synthetic words has no end-of-sequence token.
        self.eos_token_ids: tuple[int, ...] = ()

    @property
    def vocab_size(self) -> int:
        return int(self._tok.get_vocab_size())

    def encode(self, text: str) -> list[int]:
        """Token ids of `text`, without special tokens (the engine controls templating)."""
        return self._tok.encode(text, add_special_tokens=False).ids

    def decode(self, token_ids: list[int]) -> str:
        return self._tok.decode(token_ids, skip_special_tokens=True)
