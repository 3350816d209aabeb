"""Pins the oracle of the model files (oracle/model_files.py) before it is
used as the checker:
  - the index reader against an index assembled by hand, field by field
    (tools/make_index.py:3-11);
  - the pre-tokenizer against the `regex` module evaluating the split
    pattern the reference hand-codes (src/tokenizer.h:105-153), on ASCII
    text, and against pieces derived by hand from tokenizer.h where the two
    differ;
  - encode against ids the HuggingFace `tokenizers` library produced on the
    synthetic tokenizer (tests/golden/make_tok.py), and decode(encode(s))
    == s on arbitrary valid UTF-8."""
import json
import os
import random
import struct

import pytest

from oracle import model_files as om

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_read_index_hand_assembled():
    b = bytes([2, 0, 0, 0])                                   # u32 count 2
    b += bytes([5]) + b"embed" + bytes([0])                   # name, kind fp16
    b += (16).to_bytes(8, "little") + (4096).to_bytes(8, "little") + bytes(8)
    b += (2048).to_bytes(8, "little") + bytes(8)              # d0 2048, d1 0
    b += bytes([3]) + b"q.w" + bytes([1])                     # int4g
    b += (4112).to_bytes(8, "little") + (1 << 21).to_bytes(8, "little")
    b += (65536).to_bytes(8, "little")
    b += (2048).to_bytes(8, "little") + (2048).to_bytes(8, "little")
    got = om.read_index(b)
    assert got == [
        dict(name="embed", kind=0, offset=16, packed=4096, scales=0, d0=2048, d1=0),
        dict(name="q.w", kind=1, offset=4112, packed=1 << 21, scales=65536, d0=2048, d1=2048)]
    with pytest.raises(ValueError):
        om.read_index(b + b"\0")
    with pytest.raises(struct.error):
        om.read_index(b[:-1])


def _regex_pieces(text):
    import regex
    pat = json.load(open(os.path.join(GOLD, "tok_cases.json"), encoding="utf-8"))["pattern"]
    return regex.findall(pat, text)


def _oracle_pieces(text):
    cps = [ord(c) for c in text]
    return ["".join(map(chr, cps[a:b])) for a, b in om.pre_tokenize(cps)]


ASCII = ("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789"
         "      \n\n\r.,;:!?'''\"()-_/+*=#@&%$<>|[]{}~^`\\")


def test_pre_tokenize_matches_regex_on_ascii():
    rng = random.Random(3)
    for _ in range(3000):
        s = "".join(rng.choice(ASCII) for _ in range(rng.randint(1, 40)))
        assert _oracle_pieces(s) == _regex_pieces(s), repr(s)
    for s in ["'s", "'S'T'RE'Ve'm'LL'd", "'x", "a'", "'", "''s", "x'll", "1234567", "a1b2",
              " ", "  ", " \n ", "\r\n\r\n  x", "a  b", "a \n b", "  !", " !!\n\nx",
              "end  ", "!x", " 'x", "0'5"]:
        assert _oracle_pieces(s) == _regex_pieces(s), repr(s)


@pytest.mark.parametrize("text,pieces", [
    # a tab (or VT, FF) before letters: the hand-coded pattern takes only a
    # space or punctuation as the optional lead (tokenizer.h:121-124); the
    # regex's [^\r\n\p{L}\p{N}]? would take the tab too
    ("\tword", ["\t", "word"]),
    ("a\t\tb", ["a", "\t", "\t", "b"]),
    ("x\x0by", ["x", "\x0b", "y"]),
    # every non-whitespace code point >= 0x80 is a letter (tokenizer.h:95-99):
    # the euro sign and an emoji are letters
    ("a€b c", ["a€b", " c"]),
    ("\U0001F600!", ["\U0001F600", "!"]),
    ("ét", ["ét"]),
    # U+00A0 is whitespace there, and (like a tab) no lead before letters
    ("a\u00a0\u00a0b", ["a", "\u00a0", "\u00a0", "b"]),
])
def test_pre_tokenize_where_the_reference_differs_from_the_regex(text, pieces):
    assert _oracle_pieces(text) == pieces


def test_oracle_encode_matches_library_vectors():
    tok = om.Tokenizer.load(os.path.join(GOLD, "tok"))
    cases = json.load(open(os.path.join(GOLD, "tok_cases.json"), encoding="utf-8"))["cases"]
    assert len(cases) >= 70
    for c in cases:
        assert tok.encode(c["text"].encode()) == c["ids"], repr(c["text"])


def test_oracle_round_trip_and_specials():
    tok = om.Tokenizer.load(os.path.join(GOLD, "tok"))
    rng = random.Random(9)
    pool = [chr(c) for c in range(32, 127)] + list("\t\n\r\x0b\x0c éßñ中文ми€\U0001F600́")
    for _ in range(300):
        s = "".join(rng.choice(pool) for _ in range(rng.randint(0, 60)))
        ids = tok.encode(s.encode())
        assert tok.decode(ids) == s.encode(), repr(s)
    # the longer of two specials sharing a prefix wins where both match
    sp = {c: i for c, i in tok.specials}
    assert tok.encode(b"<think></think>") == [sp[b"<think></think>"]]
    assert tok.encode(b"<think></thin")[0] == sp[b"<think>"]
    assert tok.decode([sp[b"<|im_end|>"], 999999, -1], skip_special=True) == b""
