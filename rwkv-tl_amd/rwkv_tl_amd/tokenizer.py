"""RWKV "world" tokenizer: greedy longest match over a byte vocabulary.

Same API and tokenization as ``rwkv_tl.tokenizer.Tokenizer``
(``src/rwkv_tl/tokenizer.py:28-90``): ``encode`` / ``decode`` on str,
``encodeBytes`` / ``decodeBytes`` on bytes. At every position the longest
vocabulary entry that prefixes the remaining bytes is emitted; every single
byte is in the vocabulary, so any input encodes.

The vocabulary file has one entry per line, ``<id> <literal> <length>``, where
``<literal>`` is a Python str or bytes literal (a str stands for its UTF-8
bytes) and ``<length>`` its byte length (``asset/rwkv_vocab_v20230424.txt`` of
the reference). Literals are parsed with ``ast.literal_eval``, which evaluates
nothing but literals.

Host code: tokenization is not on the GPU path.
"""

from __future__ import annotations

import ast
from collections.abc import Sequence


class Tokenizer:
    def __init__(self, vocab_path: str) -> None:
        entries: dict[int, bytes] = {}
        with open(vocab_path, "r", encoding="utf-8") as f:
            for n, line in enumerate(f, 1):
                line = line.rstrip("\n")
                if not line:
                    continue
                first, last = line.index(" "), line.rindex(" ")
                idx = int(line[:first])
                lit = ast.literal_eval(line[first + 1 : last])
                tok = lit.encode("utf-8") if isinstance(lit, str) else lit
                if not isinstance(tok, bytes):
                    raise ValueError(f"{vocab_path}:{n}: entry is neither str nor bytes")
                if len(tok) != int(line[last + 1 :]):
                    raise ValueError(f"{vocab_path}:{n}: length {len(tok)} != declared {line[last + 1:]}")
                entries[idx] = tok
        self.token2idx: dict[bytes, int] = {t: i for i, t in entries.items()}
        self.idx2token: list[bytes] = [b""] * (max(entries) + 1)
        for i, t in entries.items():
            self.idx2token[i] = t
        missing = [b for b in range(256) if bytes([b]) not in self.token2idx]
        if missing:
            raise ValueError(f"{vocab_path}: single bytes {missing[:8]} missing from the vocabulary")
        # longest entry starting with each byte: the candidate lengths at a position
        self._maxlen = [1] * 256
        for t in self.token2idx:
            self._maxlen[t[0]] = max(self._maxlen[t[0]], len(t))

    def encodeBytes(self, src: bytes) -> list[int]:
        out: list[int] = []
        lookup, maxlen = self.token2idx, self._maxlen
        i, n = 0, len(src)
        while i < n:
            for L in range(min(maxlen[src[i]], n - i), 0, -1):
                idx = lookup.get(src[i : i + L])
                if idx is not None:
                    out.append(idx)
                    i += L
                    break
        return out

    def decodeBytes(self, tokens: Sequence[int]) -> bytes:
        return b"".join(self.idx2token[t] for t in tokens)

    def encode(self, src: str) -> list[int]:
        return self.encodeBytes(src.encode("utf-8"))

    def decode(self, tokens: Sequence[int]) -> str:
        return self.decodeBytes(tokens).decode("utf-8")
