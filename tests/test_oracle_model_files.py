"""Pins the oracle of the model files (oracle/model_files.py) before the
product is compared against it:
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


ref_tok = pytest.mark.skipif(not om.RefTokenizer.available(),
                             reason="oracle/_ref/libreftok.so not built (no reference tree)")


def _random_inputs(seed, n):
    rng = random.Random(seed)
    pool = ([chr(c) for c in range(32, 127)] * 3 + list("\t\n\r\x0b\x0c\xa0") +
            list("éßñ中文ми€\U0001F600́　 ٣"))
    out = []
    for _ in range(n):
        if rng.random() < 0.25:
            out.append(bytes(rng.randrange(256) for _ in range(rng.randint(0, 64))))
        else:
            out.append("".join(rng.choice(pool) for _ in range(rng.randint(0, 120))).encode())
    return out


@ref_tok
def test_oracle_matches_compiled_reference_tokenizer():
    """The oracle against src/tokenizer.h itself (compiled from the header
    where it lies): golden cases, random UTF-8 and random bytes, specials
    inserted, decode of random ids with and without skip_special."""
    d = os.path.join(GOLD, "tok")
    ref, tok = om.RefTokenizer(d), om.Tokenizer.load(d)
    cases = json.load(open(os.path.join(GOLD, "tok_cases.json"), encoding="utf-8"))["cases"]
    texts = [c["text"].encode() for c in cases] + _random_inputs(41, 500)
    specials = [c for c, _ in tok.specials]
    rng = random.Random(42)
    for t in texts:
        if rng.random() < 0.3:
            k = rng.randint(0, len(t))
            t = t[:k] + rng.choice(specials) + t[k:]
        assert tok.encode(t) == ref.encode(t), t
    nv = len(tok.id2tok)
    for _ in range(300):
        ids = [rng.randrange(-3, nv + 5) for _ in range(rng.randint(0, 40))]
        for skip in (False, True):
            assert tok.decode(ids, skip) == ref.decode(ids, skip), ids


@ref_tok
def test_oracle_matches_compiled_reference_on_degenerate_files(tmp_path):
    """Merge results missing from the vocabulary, duplicate lines, a tab
    inside B, lines without a tab.  Left out, as undefined in the reference:
    an empty special (its encode would loop forever) and a negative id (its
    load writes before the id table)."""
    tab = om.byte_table()
    vocab = [b"%d\t%s" % (i, tab[b].encode()) for i, b in enumerate(range(256))]
    vocab += [b"256\tab", b"257\tabc", b"258\txyz", b"259\tab", b"no tab line", b"260\tneg"]
    merges = [b"0\ta\tb", b"1\tab\tc", b"2\tx\ty", b"3\txy\tz", b"5\tq\tq", b"4\tc\td",
              b"7\tab\tcd", b"9\tz\tz\tz", b"x", b"6\tq\tq"]
    special = [b"300\t<s>", b"302\t<s>x", b"bad"]
    d = tmp_path / "tok"
    d.mkdir()
    for name, lines in (("vocab.tsv", vocab), ("merges.tsv", merges), ("special.tsv", special)):
        (d / name).write_bytes(b"".join(x + b"\n" for x in lines))
    ref, tok = om.RefTokenizer(str(d)), om.Tokenizer.load(str(d))
    rng = random.Random(7)
    for s in [b"abc", b"abcd", b"xyz", b"xyzz", b"qqq", b"qqqq", b"cdab", b"<s>x<s><s>y",
              b"zzz", b"ab ab", b"neg"] + [
            bytes(rng.choice(b"abcdxyzq <s>") for _ in range(rng.randint(0, 30)))
            for _ in range(300)]:
        assert tok.encode(s) == ref.encode(s), s
    ids = list(range(-2, 310))
    assert tok.decode(ids) == ref.decode(ids)
    assert tok.decode(ids, True) == ref.decode(ids, True)
