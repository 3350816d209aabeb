"""The model-file entries of include/cuda_inf_model.h on the CPU (host code:
no GPU call): the index reader and the tokenizer against the oracle
(oracle/model_files.py), bit-exact, and their error paths.

Tokenizer parity (src/tokenizer.h): the golden cases, random valid UTF-8
(tabs, NBSP, emoji, combining marks: where the reference's hand-coded
pattern departs from the textbook regex), random bytes (malformed UTF-8,
which the reference reads 4 bytes per stray lead), random id sequences for
decode (specials, out-of-range ids, skip_special), and degenerate
vocabularies (merge results missing from the vocabulary, duplicate lines,
an empty special)."""
import ctypes
import json
import os
import random

import pytest

from oracle import model_files as om

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOK = os.path.join(GOLD, "tok")


@pytest.fixture(scope="module")
def toks(cia):
    from cuda_inf_amd.model_files import Tokenizer
    t = Tokenizer()
    assert t.load(TOK)
    return t, om.Tokenizer.load(TOK)


def test_golden_cases(toks):
    t, ref = toks
    for c in json.load(open(os.path.join(GOLD, "tok_cases.json"), encoding="utf-8"))["cases"]:
        assert t.encode(c["text"]) == c["ids"], repr(c["text"])
        assert t.decode_bytes(c["ids"]) == ref.decode(c["ids"])


def test_random_text_matches_oracle(toks):
    t, ref = toks
    rng = random.Random(21)
    pool = ([chr(c) for c in range(32, 127)] * 3 + list("\t\n\r\x0b\x0c\xa0") +
            list("éßñ中文ми€\U0001F600́　 ٣"))
    specials = [c.decode() for c, _ in ref.specials]
    for _ in range(400):
        s = "".join(rng.choice(pool) for _ in range(rng.randint(0, 120)))
        if rng.random() < 0.3:
            k = rng.randint(0, len(s))
            s = s[:k] + rng.choice(specials) + s[k:]
        b = s.encode()
        ids = t.encode(b)
        assert ids == ref.encode(b), repr(s)
        assert t.decode_bytes(ids) == b, repr(s)


def test_random_bytes_match_oracle(toks):
    t, ref = toks
    rng = random.Random(22)
    for _ in range(400):
        b = bytes(rng.randrange(256) for _ in range(rng.randint(0, 64)))
        assert t.encode(b) == ref.encode(b), b


@pytest.mark.skipif(not om.RefTokenizer.available(),
                    reason="oracle/_ref/libreftok.so not built (no reference tree)")
def test_matches_compiled_reference_tokenizer(toks):
    """Directly against src/tokenizer.h compiled from the header."""
    t, _ = toks
    ref = om.RefTokenizer(TOK)
    rng = random.Random(24)
    pool = [chr(c) for c in range(32, 127)] * 3 + list("\t\n\r\xa0éß中€\U0001F600́")
    for _ in range(300):
        if rng.random() < 0.3:
            b = bytes(rng.randrange(256) for _ in range(rng.randint(0, 64)))
        else:
            b = "".join(rng.choice(pool) for _ in range(rng.randint(0, 100))).encode()
        ids = t.encode(b)
        assert ids == ref.encode(b), b
        assert t.decode_bytes(ids) == ref.decode(ids)


def test_decode_random_ids(toks):
    t, ref = toks
    rng = random.Random(23)
    nv = len(ref.id2tok)
    sp = list(ref.id2special)
    for _ in range(300):
        ids = [rng.choice(sp) if rng.random() < 0.1 else rng.randrange(-3, nv + 5)
               for _ in range(rng.randint(0, 40))]
        for skip in (False, True):
            assert t.decode_bytes(ids, skip) == ref.decode(ids, skip), (ids, skip)


def _write_tok(d, vocab_lines, merge_lines, special_lines):
    os.makedirs(d, exist_ok=True)
    for name, lines in (("vocab.tsv", vocab_lines), ("merges.tsv", merge_lines),
                        ("special.tsv", special_lines)):
        with open(os.path.join(d, name), "wb") as f:
            f.write(b"".join(x + b"\n" for x in lines))


def test_degenerate_vocabulary(cia, tmp_path):
    """Merges whose result is not a token (its symbols are dropped, as the
    reference drops them), a later duplicate line winning, merge lines with
    a tab inside B, an empty special (ignored), lines without a tab."""
    from cuda_inf_amd.model_files import Tokenizer
    tab = om.byte_table()
    chars = [tab[b].encode() for b in range(256)]
    vocab = [b"%d\t%s" % (i, c) for i, c in enumerate(chars)]
    vocab += [b"256\tab", b"257\tabc", b"258\txyz", b"259\tab", b"no tab line", b"-4\tneg"]
    merges = [b"0\ta\tb", b"1\tab\tc", b"2\tx\ty", b"3\txy\tz", b"5\tq\tq",
              b"4\tc\td", b"7\tab\tcd", b"9\tz\tz\tz", b"x", b"6\tq\tq"]
    special = [b"300\t<s>", b"301\t", b"302\t<s>x", b"bad"]
    d = str(tmp_path / "tok")
    _write_tok(d, vocab, merges, special)
    t = Tokenizer()
    assert t.load(d)
    ref = om.Tokenizer.load(d)
    rng = random.Random(4)
    for s in [b"abc", b"abcd", b"xyz", b"xyzz", b"qqq", b"qqqq", b"cdab", b"<s>x<s><s>y",
              b"zzz", b"ab ab", b"neg"] + [
            bytes(rng.choice(b"abcdxyzq <s>") for _ in range(rng.randint(0, 30)))
            for _ in range(200)]:
        assert t.encode(s) == ref.encode(s), s
    ids = list(range(-2, 310))
    assert t.decode_bytes(ids) == ref.decode(ids)
    assert t.decode_bytes(ids, True) == ref.decode(ids, True)


def test_tokenizer_errors(cia, tmp_path):
    from cuda_inf_amd import _lib
    from cuda_inf_amd.model_files import Tokenizer
    t = Tokenizer()
    assert not t.load(str(tmp_path / "missing"))
    with pytest.raises(RuntimeError):
        t.encode("x")
    L = _lib.lib()
    h = ctypes.c_void_p()
    assert L.cia_tok_load(None, ctypes.byref(h)) == 1
    assert L.cia_tok_load(TOK.encode(), ctypes.byref(h)) == 0 and h.value
    n = ctypes.c_int64()
    text = b"hello world, again and again"
    assert L.cia_tok_encode(h, text, len(text), None, 0, ctypes.byref(n)) == 0 and n.value > 1
    small = (ctypes.c_int32 * 1)()
    assert L.cia_tok_encode(h, text, len(text), small, 1, ctypes.byref(n)) == 3
    assert L.cia_tok_encode(h, text, -1, small, 1, ctypes.byref(n)) == 3
    assert L.cia_tok_encode(h, None, 0, small, 1, ctypes.byref(n)) == 0 and n.value == 0
    ids = (ctypes.c_int32 * 3)(40, 41, 42)
    assert L.cia_tok_decode(h, ids, 3, 0, None, 0, ctypes.byref(n)) == 0 and n.value == 3
    buf = ctypes.create_string_buffer(2)
    assert L.cia_tok_decode(h, ids, 3, 0, buf, 2, ctypes.byref(n)) == 3
    assert L.cia_tok_decode(h, None, 1, 0, None, 0, ctypes.byref(n)) == 1
    L.cia_tok_free(h)
    L.cia_tok_free(None)


def _index_records(rng, n):
    out = []
    off = 0
    for i in range(n):
        kind = rng.randrange(2)
        name = "model.layers.%d.%s" % (i, rng.choice(["self_attn.q_proj.weight", "norm", "x" * 200]))
        d0, d1 = rng.randrange(1, 4096), (rng.randrange(1, 32) * 128 if kind else rng.choice([0, 64]))
        packed = d0 * d1 // 2 if kind else 2 * d0 * max(d1, 1)
        scales = d0 * (d1 // 128) * 2 if kind else 0
        out.append(dict(name=name, kind=kind, offset=off, packed=packed, scales=scales, d0=d0, d1=d1))
        off += packed + scales
    return out


def test_index_read_matches_oracle(cia, tmp_path):
    from cuda_inf_amd.model_files import TensorDesc, read_index
    rng = random.Random(5)
    recs = _index_records(rng, 300)
    p = str(tmp_path / "index.bin")
    om.write_index(p, recs)
    got = read_index(p)
    ref = om.read_index(p)
    assert list(got) == [r["name"] for r in ref]
    for r in ref:
        assert got[r["name"]] == TensorDesc(r["kind"], r["offset"], r["packed"], r["scales"],
                                            r["d0"], r["d1"])
    # empty index
    om.write_index(p, [])
    assert read_index(p) == {}


def test_index_read_errors(cia, tmp_path):
    from cuda_inf_amd import _lib
    L = _lib.lib()
    p = str(tmp_path / "index.bin")
    om.write_index(p, _index_records(random.Random(6), 3))
    good = open(p, "rb").read()
    n = ctypes.c_int64()
    arr = (_lib.cia_tensor_desc * 3)()
    assert L.cia_index_read(p.encode(), None, 0, ctypes.byref(n)) == 0 and n.value == 3
    assert L.cia_index_read(p.encode(), arr, 2, ctypes.byref(n)) == 3
    assert L.cia_index_read(p.encode(), arr, 3, ctypes.byref(n)) == 0
    assert L.cia_index_read(str(tmp_path / "none").encode(), arr, 3, ctypes.byref(n)) == 7
    assert L.cia_index_read(None, arr, 3, ctypes.byref(n)) == 1
    bad_kind = bytearray(good)
    bad_kind[4 + 1 + good[4]] = 2  # first record's kind byte
    for data in (good[:-1], good + b"\0", bytes(bad_kind), b"", b"\1\0\0"):
        with open(p, "wb") as f:
            f.write(data)
        assert L.cia_index_read(p.encode(), arr, 3, ctypes.byref(n)) == 7, data[:8]
    u = ctypes.c_uint64()
    assert L.cia_file_size(str(tmp_path).encode(), ctypes.byref(u)) == 7  # a directory
    assert L.cia_file_size(p.encode(), ctypes.byref(u)) == 0 and u.value == 3
    # upload argument checks that return before any device call
    assert L.cia_weights_upload(None, 0x10000, 8, ctypes.byref(u), None) == 1
    assert L.cia_weights_upload(str(tmp_path / "none").encode(), 0x10000, 8,
                                ctypes.byref(u), None) == 7
    assert L.cia_weights_upload(p.encode(), 0x10000, 2, ctypes.byref(u), None) == 3
