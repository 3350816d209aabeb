"""CPU restatement of the reference's model-file handling: the weight index
reader and the byte-level BPE tokenizer, in plain Python.

TEST INFRASTRUCTURE ONLY: the product is compared against it.  Only tests/ import
this module; the product (cuda_inf_amd, include/cuda_inf_model.h) never does.

Pinned by tests/test_oracle_model_files.py:
  - read_index: a hand-assembled index (every field spelled out in bytes).
  - pre_tokenize: the `regex` module's evaluation of the pattern the
    reference hand-codes, on ASCII text (where its letter/space classes are
    the regex's), plus hand-derived pieces for the inputs where the two
    differ (a tab before letters; non-ASCII punctuation counted as a letter).
  - encode / decode: the HuggingFace `tokenizers` library (BPE with
    ignore_merges, the same split pattern, byte-level mapping) on a
    tokenizer trained from synthetic text; decode(encode(s)) == s;
  - and, where the reference tree is present, src/tokenizer.h itself:
    oracle/Makefile compiles the header where it lies (with ref_tok.cpp, a
    C-ABI shim) into oracle/_ref/libreftok.so, and ``RefTokenizer`` calls
    it; encode and decode agree on the golden cases, random text and bytes,
    random ids and degenerate files.
"""
from __future__ import annotations

import os
import struct

# ---------------------------------------------------------------- index.bin


def read_index(path_or_bytes) -> list[dict]:
    """index.bin -> list of tensor records (tools/make_index.py:3-11, read
    as src/engine.cu:665-675 reads it)."""
    if isinstance(path_or_bytes, (bytes, bytearray)):
        b = bytes(path_or_bytes)
    else:
        with open(path_or_bytes, "rb") as f:
            b = f.read()
    (n,) = struct.unpack_from("<I", b, 0)
    p = 4
    out = []
    for _ in range(n):
        nl = b[p]
        name = b[p + 1:p + 1 + nl].decode("utf-8", "surrogateescape")
        p += 1 + nl
        kind, off, packed, scales, d0, d1 = struct.unpack_from("<BQQQqq", b, p)
        p += 1 + 8 * 5
        out.append(dict(name=name, kind=kind, offset=off, packed=packed, scales=scales,
                        d0=d0, d1=d1))
    if p != len(b):
        raise ValueError("trailing bytes")
    return out


def write_index(path: str, tensors: list[dict]) -> None:
    """The inverse (tools/make_index.py:24-36), for building test files."""
    with open(path, "wb") as o:
        o.write(struct.pack("<I", len(tensors)))
        for t in tensors:
            nm = t["name"].encode()
            o.write(struct.pack("<B", len(nm)) + nm)
            o.write(struct.pack("<BQQQqq", t["kind"], t["offset"], t["packed"], t["scales"],
                                t["d0"], t["d1"]))


# ---------------------------------------------------------------- tokenizer


def byte_table() -> list[str]:
    """byte -> byte-level character (src/tokenizer.h:30-41)."""
    keep = list(range(33, 127)) + list(range(161, 173)) + list(range(174, 256))
    m = {b: b for b in keep}
    n = 0
    for b in range(256):
        if b not in m:
            m[b] = 256 + n
            n += 1
    return [chr(m[b]) for b in range(256)]


def to_cps(raw: bytes) -> list[int]:
    """src/tokenizer.h:83-92 (including its reading of malformed UTF-8)."""
    cps, i, n = [], 0, len(raw)
    while i < n:
        c = raw[i]
        if c < 0x80:
            cp, k = c, 1
        elif (c >> 5) == 0x6:
            cp, k = c & 0x1F, 2
        elif (c >> 4) == 0xE:
            cp, k = c & 0xF, 3
        else:
            cp, k = c & 0x7, 4
        j = 1
        while j < k and i + j < n:
            cp = (cp << 6) | (raw[i + j] & 0x3F)
            j += 1
        cps.append(cp)
        i += k
    return cps


def cp_to_utf8(cp: int) -> bytes:
    """src/tokenizer.h:24-29 (no range check: any 21-bit value)."""
    if cp < 0x80:
        return bytes([cp])
    if cp < 0x800:
        return bytes([0xC0 | (cp >> 6), 0x80 | (cp & 0x3F)])
    if cp < 0x10000:
        return bytes([0xE0 | (cp >> 12), 0x80 | ((cp >> 6) & 0x3F), 0x80 | (cp & 0x3F)])
    return bytes([0xF0 | (cp >> 18), 0x80 | ((cp >> 12) & 0x3F), 0x80 | ((cp >> 6) & 0x3F),
                  0x80 | (cp & 0x3F)])


def _is_ws(c):  # src/tokenizer.h:93
    return c in (0x20, 0x09, 0x0A, 0x0D, 0x0B, 0x0C, 0xA0)


def _is_digit(c):  # :94
    return 0x30 <= c <= 0x39


def _is_letter(c):  # :95-99
    return (0x41 <= c <= 0x5A) or (0x61 <= c <= 0x7A) or (c >= 0x80 and not _is_ws(c))


def _is_punct(c):  # :100
    return not _is_ws(c) and not _is_letter(c) and not _is_digit(c)


def _lower(c):  # :102
    return c + 32 if 0x41 <= c <= 0x5A else c


def pre_tokenize(c: list[int]) -> list[tuple[int, int]]:
    """Piece ranges [start, end) over code points (src/tokenizer.h:105-153)."""
    n, out, i = len(c), [], 0
    while i < n:
        # contraction (:107-118)
        m = 0
        if c[i] == 0x27 and i + 1 < n:
            a = _lower(c[i + 1])
            if a in (0x73, 0x74, 0x6D, 0x64):
                m = 2
            elif i + 2 < n:
                b = _lower(c[i + 2])
                if (a, b) in ((0x72, 0x65), (0x76, 0x65), (0x6C, 0x6C)):
                    m = 3
        if m:
            out.append((i, i + m))
            i += m
            continue
        # letters; one non-letter/digit/ws then letters; a space then letters (:120-124)
        if _is_letter(c[i]):
            j = i
            while j < n and _is_letter(c[j]):
                j += 1
            out.append((i, j))
            i = j
            continue
        if (not _is_digit(c[i]) and c[i] not in (0x0D, 0x0A) and not _is_ws(c[i])
                and i + 1 < n and _is_letter(c[i + 1])):
            j = i + 1
            while j < n and _is_letter(c[j]):
                j += 1
            out.append((i, j))
            i = j
            continue
        if c[i] == 0x20 and i + 1 < n and _is_letter(c[i + 1]):
            j = i + 1
            while j < n and _is_letter(c[j]):
                j += 1
            out.append((i, j))
            i = j
            continue
        # 1-3 digits (:125-126)
        if _is_digit(c[i]):
            j = i
            while j < n and _is_digit(c[j]) and j - i < 3:
                j += 1
            out.append((i, j))
            i = j
            continue
        # optional space, punctuation, then CR/LF (:127-137)
        p = i + 1 if c[i] == 0x20 else i
        if p < n and _is_punct(c[p]):
            q = p
            while q < n and _is_punct(c[q]):
                q += 1
            while q < n and c[q] in (0x0D, 0x0A):
                q += 1
            out.append((i, q))
            i = q
            continue
        # whitespace (:138-148)
        if _is_ws(c[i]):
            e = i
            while e < n and _is_ws(c[e]):
                e += 1
            last = -1
            for k in range(i, e):
                if c[k] in (0x0D, 0x0A):
                    last = k
            if last >= 0:
                end = last + 1
            elif e == n:
                end = e
            elif e - 1 > i:
                end = e - 1
            else:
                end = e
            out.append((i, end))
            i = end
            continue
        out.append((i, i + 1))  # (:149-150)
        i += 1
    return out


def _u8_split(s: bytes) -> list[bytes]:
    """UTF-8 characters of a byte string by lead byte (src/tokenizer.h:159-162)."""
    out, i = [], 0
    while i < len(s):
        ch = s[i]
        k = 1 if ch < 0x80 else (2 if (ch >> 5) == 0x6 else (3 if (ch >> 4) == 0xE else 4))
        out.append(s[i:i + k])
        i += k
    return out


class Tokenizer:
    """src/tokenizer.h:15-232, restated over bytes (a token string is the
    UTF-8 bytes of its byte-level form)."""

    def __init__(self, vocab: dict[bytes, int], id2tok: list[bytes],
                 merges: dict[tuple[bytes, bytes], int], specials: list[tuple[bytes, int]],
                 id2special: dict[int, bytes]):
        self.vocab, self.id2tok, self.merges = vocab, id2tok, merges
        # longest first (:77; equal lengths keep file order)
        self.specials = sorted([s for s in specials if s[0]], key=lambda x: -len(x[0]))
        self.id2special = id2special
        self.b2u = [ch.encode() for ch in byte_table()]
        self.u2b = {u: b for b, u in enumerate(self.b2u)}

    @classmethod
    def load(cls, d: str) -> "Tokenizer":
        """src/tokenizer.h:42-81."""
        def lines(name):
            with open(os.path.join(d, name), "rb") as f:
                data = f.read()
            out = data.split(b"\n")
            if out and out[-1] == b"":
                out.pop()
            return out
        vocab, tmp, maxid = {}, [], 0
        for ln in lines("vocab.tsv"):
            if b"\t" not in ln:
                continue
            a, s = ln.split(b"\t", 1)
            i = int(a)
            tmp.append((i, s))
            vocab[s] = i
            maxid = max(maxid, i)
        id2tok = [b""] * (maxid + 1)
        for i, s in tmp:
            if i >= 0:
                id2tok[i] = s
        merges = {}
        for ln in lines("merges.tsv"):
            parts = ln.split(b"\t", 2)
            if len(parts) < 3:
                continue
            merges[(parts[1], parts[2])] = int(parts[0])
        specials, id2special = [], {}
        for ln in lines("special.tsv"):
            if b"\t" not in ln:
                continue
            a, s = ln.split(b"\t", 1)
            specials.append((s, int(a)))
            id2special[int(a)] = s
        return cls(vocab, id2tok, merges, specials, id2special)

    def bpe_word(self, word: bytes, out: list[int]) -> None:
        """src/tokenizer.h:155-175."""
        if word in self.vocab:
            out.append(self.vocab[word])
            return
        syms = _u8_split(word)
        while len(syms) > 1:
            best, at = None, -1
            for j in range(len(syms) - 1):
                r = self.merges.get((syms[j], syms[j + 1]))
                if r is not None and (best is None or r < best):
                    best, at = r, j
            if at < 0:
                break
            syms[at:at + 2] = [syms[at] + syms[at + 1]]
        out.extend(self.vocab[s] for s in syms if s in self.vocab)

    def pieces(self, text: bytes) -> list[bytes]:
        """Raw bytes of each pre-tokenized piece of a special-free chunk."""
        cps = to_cps(text)
        return [b"".join(cp_to_utf8(c) for c in cps[a:b]) for a, b in pre_tokenize(cps)]

    def encode(self, text: bytes) -> list[int]:
        """src/tokenizer.h:177-208."""
        out, pos, n = [], 0, len(text)
        while pos < n:
            best_pos, best_id, best_len = -1, -1, 0
            for s, i in self.specials:
                f = text.find(s, pos)
                if f >= 0 and (best_pos < 0 or f < best_pos or (f == best_pos and len(s) > best_len)):
                    best_pos, best_id, best_len = f, i, len(s)
            end = n if best_pos < 0 else best_pos
            if end > pos:
                for raw in self.pieces(text[pos:end]):
                    self.bpe_word(b"".join(self.b2u[b] for b in raw), out)
            if best_pos < 0:
                break
            out.append(best_id)
            pos = best_pos + best_len
        return out

    def _bl_to_raw(self, bl: bytes) -> bytes:  # :212-217
        return bytes(self.u2b[ch] for ch in _u8_split(bl) if ch in self.u2b)

    def decode(self, ids, skip_special: bool = False) -> bytes:
        """src/tokenizer.h:218-231."""
        out, bl = b"", b""
        for i in ids:
            if i in self.id2special:
                out += self._bl_to_raw(bl)
                bl = b""
                if not skip_special:
                    out += self.id2special[i]
                continue
            if 0 <= i < len(self.id2tok):
                bl += self.id2tok[i]
        return out + self._bl_to_raw(bl)


# ------------------------------------------------ the reference's tokenizer

REF_TOK_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_ref", "libreftok.so")


class RefTokenizer:
    """src/tokenizer.h itself, compiled by oracle/Makefile into
    oracle/_ref/libreftok.so (present only where the reference tree was
    available at build time; ``available()`` says so)."""

    _lib = None

    @classmethod
    def available(cls) -> bool:
        return os.path.exists(REF_TOK_LIB)

    @classmethod
    def _l(cls):
        import ctypes
        if cls._lib is None:
            L = ctypes.CDLL(REF_TOK_LIB)
            P, I64 = ctypes.c_void_p, ctypes.c_int64
            L.ref_tok_load.restype, L.ref_tok_load.argtypes = P, [ctypes.c_char_p]
            L.ref_tok_free.restype, L.ref_tok_free.argtypes = None, [P]
            L.ref_tok_encode.restype = I64
            L.ref_tok_encode.argtypes = [P, ctypes.c_char_p, I64, P, I64]
            L.ref_tok_decode.restype = I64
            L.ref_tok_decode.argtypes = [P, P, I64, ctypes.c_int, P, I64]
            cls._lib = L
        return cls._lib

    def __init__(self, d: str):
        self.h = self._l().ref_tok_load(os.fsencode(d))
        if not self.h:
            raise FileNotFoundError(d)

    def __del__(self):
        if getattr(self, "h", None):
            self._l().ref_tok_free(self.h)

    def encode(self, text: bytes) -> list[int]:
        import ctypes
        buf = (ctypes.c_int32 * max(len(text), 1))()
        n = self._l().ref_tok_encode(self.h, text, len(text), buf, len(text))
        return list(buf[:n])

    def decode(self, ids, skip_special: bool = False) -> bytes:
        import ctypes
        ids = list(ids)
        arr = (ctypes.c_int32 * max(len(ids), 1))(*ids)
        n = self._l().ref_tok_decode(self.h, arr, len(ids), int(skip_special), None, 0)
        out = ctypes.create_string_buffer(max(n, 1))
        self._l().ref_tok_decode(self.h, arr, len(ids), int(skip_special), out, n)
        return out.raw[:n]
