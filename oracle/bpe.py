"""Byte-level BPE restated in plain Python: AccelEP's accel::Bpe (src/bpe.cc). TEST
INFRASTRUCTURE ONLY: the tests compare the library's tokenizer (accelep_amd/csrc/tokenizer.cc,
through accel_llama_encode / decode / complete) with this; nothing in the library imports it.

Pinned by tests/test_tokenizer.py against
* Hugging Face `tokenizers` (the truth AccelEP's own test uses, tests/test_serve.py:182-234)
  on the fixture tokenizer and the strings of tests/golden/tokenizer_cases.json, for encode
  and for decodes whose bytes are valid UTF-8;
* the compiled reference (oracle/_ref, src/bpe.cc itself) on the same strings, on random
  byte strings and on random id lists, including decodes of invalid UTF-8;
* unicodedata for the letter and number classes, and the reference's own class tables.
"""

from __future__ import annotations

import json
import unicodedata


def byte_alphabet():
    """GPT-2's byte -> code point table (src/bpe.cc:465-502): the bytes '!'..'~', 0xA1..0xAC
    and 0xAE..0xFF stand for themselves; the other 68 take 256, 257, ... in byte order."""
    keep = set(range(0x21, 0x7F)) | set(range(0xA1, 0xAD)) | set(range(0xAE, 0x100))
    table = {}
    extra = 0
    for b in range(256):
        if b in keep:
            table[b] = b
        else:
            table[b] = 256 + extra
            extra += 1
    return table


def is_letter(cp: int) -> bool:
    """\\p{L} (src/bpe.cc:338, tables src/unicode_cats.inc)."""
    return unicodedata.category(chr(cp)).startswith("L")


def is_number(cp: int) -> bool:
    """\\p{N} (src/bpe.cc:339)."""
    return unicodedata.category(chr(cp)).startswith("N")


SPACES = frozenset([0x09, 0x0A, 0x0B, 0x0C, 0x0D, 0x20, 0x85, 0xA0, 0x1680, *range(0x2000, 0x200B), 0x2028, 0x2029,
                    0x202F, 0x205F, 0x3000])


def is_space(cp: int) -> bool:
    """\\s, the White_Space property (src/bpe.cc:341-345)."""
    return cp in SPACES


def is_other(cp: int) -> bool:
    """[^\\s\\p{L}\\p{N}] (src/bpe.cc:410)."""
    return not is_space(cp) and not is_letter(cp) and not is_number(cp)


def utf8_at(data: bytes, i: int):
    """(code point, length) of the shortest-form UTF-8 sequence at data[i], or None
    (src/bpe.cc:53-94: no overlongs, surrogates or values above U+10FFFF)."""
    c = data[i]
    if c < 0x80:
        return c, 1
    if c & 0xE0 == 0xC0:
        need, value, least = 2, c & 0x1F, 0x80
    elif c & 0xF0 == 0xE0:
        need, value, least = 3, c & 0x0F, 0x800
    elif c & 0xF8 == 0xF0:
        need, value, least = 4, c & 0x07, 0x10000
    else:
        return None
    if i + need > len(data):
        return None
    for k in range(1, need):
        if data[i + k] & 0xC0 != 0x80:
            return None
        value = (value << 6) | (data[i + k] & 0x3F)
    if value > 0x10FFFF or 0xD800 <= value <= 0xDFFF or value < least:
        return None
    return value, need


def lossy_utf8(data: bytes) -> str:
    """Valid sequences as they are, U+FFFD for every other byte, one per byte
    (src/bpe.cc:96-111)."""
    out = []
    i = 0
    while i < len(data):
        got = utf8_at(data, i)
        if got is None:
            out.append("�")
            i += 1
        else:
            out.append(chr(got[0]))
            i += got[1]
    return "".join(out)


def match_at(cps, i: int, limit: int) -> int:
    """End of the GPT-2 pattern's match at cps[i] within cps[:limit] (src/bpe.cc:371-462):
    's|'t|'re|'ve|'m|'ll|'d, then ' ?' + a run of letters, of numbers, of other characters,
    then \\s+(?!\\S), then \\s+."""
    for word in ("'re", "'ve", "'ll", "'s", "'t", "'m", "'d"):
        if i + len(word) <= limit and all(cps[i + k] == ord(word[k]) for k in range(len(word))):
            return i + len(word)
    for kind in (is_letter, is_number, is_other):
        j = i + 1 if cps[i] == 0x20 and i + 1 < limit and kind(cps[i + 1]) else i
        if j < limit and kind(cps[j]):
            while j < limit and kind(cps[j]):
                j += 1
            return j
    j = i
    while j < limit and is_space(cps[j]):
        j += 1
    if j == limit:
        return j
    if j - i >= 2:
        return j - 1
    return j  # \s+ (one space followed by a non-space)


class Bpe:
    """accel::Bpe (include/accel/bpe.h, src/bpe.cc)."""

    def __init__(self, path):
        doc = json.loads(open(path, encoding="utf-8").read())
        model = doc["model"]
        assert doc["normalizer"] is None and doc["post_processor"] is None and model["type"] == "BPE"
        self.vocab = dict(model["vocab"])
        self.tokens = [None] * len(self.vocab)
        for token, i in self.vocab.items():
            self.tokens[i] = token
        assert None not in self.tokens
        self.special = {a["id"] for a in doc.get("added_tokens") or [] if a.get("special")}
        self.added = [(a["content"], a["id"]) for a in doc.get("added_tokens") or []]
        alphabet = byte_alphabet()
        self.byte_symbol = {b: chr(cp) for b, cp in alphabet.items()}
        self.symbol_byte = {chr(cp): b for b, cp in alphabet.items()}
        self.byte_id = {b: self.vocab.get(sym) for b, sym in self.byte_symbol.items()}
        # src/bpe.cc:889-905: rank by position; a repeated pair keeps its lowest rank.
        self.ranks = {}
        for rank, m in enumerate(model["merges"]):
            left, right = m.split(" ") if isinstance(m, str) else m
            key = (self.vocab[left], self.vocab[right])
            if key not in self.ranks:
                self.ranks[key] = (rank, self.vocab[left + right])

    def _added_at(self, data: bytes, pos: int):
        """Longest added token at data[pos], the earliest listed on a tie (src/bpe.cc:912-929)."""
        best, best_id = 0, -1
        for text, i in self.added:
            t = text.encode("utf-8")
            if len(t) > best and data.startswith(t, pos):
                best, best_id = len(t), i
        return best, best_id

    def _merge(self, symbols):
        """Apply the lowest-ranked merge, leftmost on a tie, until none applies
        (src/bpe.cc:931-954)."""
        sym = list(symbols)
        while len(sym) >= 2:
            best = None
            for n in range(len(sym) - 1):
                hit = self.ranks.get((sym[n], sym[n + 1]))
                if hit is not None and (best is None or hit[0] < best[0]):
                    best = (hit[0], n, hit[1])
            if best is None:
                break
            _, n, joined = best
            sym[n:n + 2] = [joined]
        return sym

    def _piece(self, data: bytes):
        """src/bpe.cc:956-997: the digit split, the pattern, the byte symbols, the merges."""
        cps, starts = [], []
        i = 0
        while i < len(data):
            got = utf8_at(data, i)
            if got is None:
                raise ValueError("prompt is not utf-8")
            cps.append(got[0])
            starts.append(i)
            i += got[1]
        starts.append(len(data))
        out = []
        cursor = 0
        while cursor < len(cps):
            run = cursor + 1
            if not is_number(cps[cursor]):
                while run < len(cps) and not is_number(cps[run]):
                    run += 1
            at = cursor
            while at < run:
                end = match_at(cps, at, run)
                symbols = [self.byte_id[b] for b in data[starts[at]:starts[end]] if self.byte_id[b] is not None]
                if symbols:
                    out += self._merge(symbols)
                at = end
            cursor = run
        return out

    def encode(self, data) -> list:
        """src/bpe.cc:999-1026."""
        if isinstance(data, str):
            data = data.encode("utf-8")
        out = []
        pos = 0
        while pos < len(data):
            taken, i = self._added_at(data, pos)
            if taken:
                out.append(i)
                pos += taken
                continue
            gap = pos + 1
            while gap < len(data) and self._added_at(data, gap)[0] == 0:
                gap += 1
            out += self._piece(data[pos:gap])
            pos = gap
        return out

    def decode_bytes(self, ids, skip_special: bool) -> bytes:
        """The joined bytes before the lossy UTF-8 step (src/bpe.cc:1028-1064)."""
        out = bytearray()
        for i in ids:
            if not 0 <= i < len(self.tokens):
                raise ValueError("token id is outside the vocabulary")
            if skip_special and i in self.special:
                continue
            token = self.tokens[i]
            if all(ch in self.symbol_byte for ch in token):
                out += bytes(self.symbol_byte[ch] for ch in token)
            else:
                out += token.encode("utf-8")
        return bytes(out)

    def decode(self, ids, skip_special: bool = True) -> str:
        """src/bpe.cc:1028-1066."""
        return lossy_utf8(self.decode_bytes(ids, skip_special))
