"""Tokenizers for ``MegakernelEngine.generate`` without a network.

The reference builds its tokenizer with
``AutoTokenizer.from_pretrained("Qwen/Qwen3-0.6B")`` (/root/reference/host/weight_loader.py:48-60),
a Hub download.  Here:

* ``load_tokenizer(model_dir)`` reads the ``tokenizer.json`` of a LOCAL
  checkpoint directory (the one ``weights.convert_safetensors`` converts) with
  the ``tokenizers`` library, and its end-of-sequence id from
  ``generation_config.json`` / ``config.json`` / ``tokenizer_config.json``;
* ``ByteTokenizer`` is a self-contained UTF-8 byte tokenizer for the synthetic
  models of the tests and benchmarks (ids 0..255 are bytes, then BOS / EOS).

Both expose what the engine uses (``encode``, ``decode(ids,
skip_special_tokens)``, ``eos_token_id``), the interface of a transformers
tokenizer.
"""
from __future__ import annotations

import json
import os


class ByteTokenizer:
    """UTF-8 bytes as token ids 0..255; BOS = 256, EOS = 257 unless given."""

    def __init__(self, vocab: int = 1024, eos_token_id: int | None = None, bos_token_id: int | None = None):
        if vocab < 258:
            raise ValueError("ByteTokenizer needs a vocabulary of at least 258 ids")
        self.vocab = vocab
        self.bos_token_id = 256 if bos_token_id is None else bos_token_id
        self.eos_token_id = 257 if eos_token_id is None else eos_token_id

    def encode(self, text: str, add_bos: bool = False) -> list[int]:
        ids = list(text.encode("utf-8"))
        return [self.bos_token_id] + ids if add_bos else ids

    def decode(self, ids, skip_special_tokens: bool = False) -> str:
        out = bytearray()
        for i in ids:
            i = int(i)
            if i < 256:
                out.append(i)
            elif not skip_special_tokens:
                out += f"<|{i}|>".encode()
        return out.decode("utf-8", errors="replace")


class _LocalTokenizer:
    """A ``tokenizers.Tokenizer`` with the transformers-style surface."""

    def __init__(self, tok, eos_token_id: int | None):
        self._tok = tok
        self.eos_token_id = eos_token_id

    def encode(self, text: str) -> list[int]:
        return list(self._tok.encode(text).ids)

    def decode(self, ids, skip_special_tokens: bool = False) -> str:
        return self._tok.decode([int(i) for i in ids], skip_special_tokens=skip_special_tokens)


def _eos_from_files(model_dir: str, tok) -> int | None:
    for name, key in (("generation_config.json", "eos_token_id"), ("config.json", "eos_token_id")):
        path = os.path.join(model_dir, name)
        if os.path.exists(path):
            with open(path) as f:
                v = json.load(f).get(key)
            if isinstance(v, list):
                v = v[0] if v else None
            if v is not None:
                return int(v)
    path = os.path.join(model_dir, "tokenizer_config.json")
    if os.path.exists(path):
        with open(path) as f:
            v = json.load(f).get("eos_token")
        if isinstance(v, dict):
            v = v.get("content")
        if isinstance(v, str):
            return tok.token_to_id(v)
    return None


def load_tokenizer(model_dir: str):
    """The tokenizer of a local checkpoint directory (``tokenizer.json``)."""
    from tokenizers import Tokenizer

    path = os.path.join(model_dir, "tokenizer.json")
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} not found (a local tokenizer.json is needed; nothing is downloaded)")
    tok = Tokenizer.from_file(path)
    return _LocalTokenizer(tok, _eos_from_files(model_dir, tok))
