"""Tokenizer: greedy longest match over a byte vocabulary
(src/rwkv_tl/tokenizer.py:28-90), checked on a synthetic vocabulary in the
reference's file format against a brute-force restatement of the rule."""

from __future__ import annotations

import random

import pytest

from rwkv_tl_amd.tokenizer import Tokenizer


def _write_vocab(path, extra):
    """All 256 single bytes (ids 1..256, as the reference vocabulary), then
    `extra` multi-byte entries; str entries for printable ASCII, bytes
    literals otherwise, as in asset/rwkv_vocab_v20230424.txt."""
    lines = []
    for b in range(256):
        tok = bytes([b])
        lit = repr(tok.decode("latin-1")) if 32 <= b < 127 else repr(tok)
        lines.append(f"{b + 1} {lit} 1")
    for i, tok in enumerate(extra):
        try:
            lit = repr(tok.decode("utf-8"))
        except UnicodeDecodeError:
            lit = repr(tok)
        lines.append(f"{257 + i} {lit} {len(tok)}")
    path.write_text("\n".join(lines) + "\n", encoding="utf-8")


EXTRA = [b"th", b"the", b"there", b"he", b"ere", b" the", b"in", b"ing", b" in", b"\xe4\xbd\xa0", b"\xe4\xbd\xa0\xe5\xa5\xbd", b"\xff\xfe"]


@pytest.fixture()
def tok(tmp_path):
    p = tmp_path / "vocab.txt"
    _write_vocab(p, EXTRA)
    return Tokenizer(str(p))


def _brute(tok, src: bytes):
    """Longest vocabulary entry prefixing the rest, at every position."""
    out, i = [], 0
    while i < len(src):
        best = max((L for L in range(1, len(src) - i + 1) if src[i:i + L] in tok.token2idx))
        out.append(tok.token2idx[src[i:i + best]])
        i += best
    return out


def test_known_answers(tok):
    ids = tok.encode("there the thing")
    assert [tok.idx2token[i] for i in ids] == [b"there", b" the", b" ", b"th", b"ing"]
    assert tok.decode(ids) == "there the thing"
    assert tok.encode("你好你") == [tok.token2idx[b"\xe4\xbd\xa0\xe5\xa5\xbd"], tok.token2idx[b"\xe4\xbd\xa0"]]


def test_matches_brute_force_and_round_trips(tok):
    rng = random.Random(0)
    alphabet = [b"t", b"h", b"e", b"r", b" ", b"i", b"n", b"g", b"\xe4\xbd\xa0", b"\xff", b"\xfe", b"x"]
    for _ in range(200):
        src = b"".join(rng.choice(alphabet) for _ in range(rng.randint(0, 40)))
        ids = tok.encodeBytes(src)
        assert ids == _brute(tok, src)
        assert tok.decodeBytes(ids) == src


def test_rejects_bad_vocab(tmp_path):
    p = tmp_path / "bad.txt"
    p.write_text("1 'a' 2\n", encoding="utf-8")  # declared length wrong
    with pytest.raises(ValueError):
        Tokenizer(str(p))
    p.write_text("1 'a' 1\n", encoding="utf-8")  # single bytes missing
    with pytest.raises(ValueError):
        Tokenizer(str(p))
    p.write_text("1 __import__('os') 1\n", encoding="utf-8")  # not a literal: never evaluated
    with pytest.raises(ValueError):
        Tokenizer(str(p))


_REF_VOCAB = "/root/reference/asset/rwkv_vocab_v20230424.txt"


@pytest.mark.skipif(not __import__("os").path.exists(_REF_VOCAB), reason="reference vocabulary not present")
def test_reference_vocabulary():
    """The reference's own vocabulary file (data, read as text): every entry
    parses, has its declared length, and encodes to exactly its own id (it is
    the longest entry prefixing itself); mixed text matches the brute-force
    longest-match rule and round-trips."""
    tok = Tokenizer(_REF_VOCAB)
    assert len(tok.token2idx) == 65529
    for t, i in tok.token2idx.items():
        assert tok.encodeBytes(t) == [i]
    rng = random.Random(1)
    pieces = ["The quick brown fox", " jumps", "\n\n", "User: ", "Assistant:", "你好，世界", "🙂", "\t", "1234567"]
    for _ in range(50):
        src = "".join(rng.choice(pieces) for _ in range(rng.randint(1, 12))).encode("utf-8")
        ids = tok.encodeBytes(src)
        assert ids == _brute(tok, src)
        assert tok.decodeBytes(ids) == src
