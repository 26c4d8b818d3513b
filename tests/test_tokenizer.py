"""The byte-level BPE (accelep_amd/csrc/tokenizer.cc, behind accel_llama_tokenizer / encode /
decode / complete) on the CPU.

The oracle (oracle/bpe.py, a restatement of AccelEP's src/bpe.cc) is pinned first:
* its byte alphabet and lossy UTF-8 step by closed forms;
* its pattern split against the `regex` module running GPT-2's pattern itself;
* its letter/number classes against unicodedata and the reference's own tables;
* its encode and decode against Hugging Face `tokenizers` (what AccelEP's tokenizer test
  checks against, tests/test_serve.py:182-234) on the fixture strings and on seeded random
  strings, and against the compiled reference (oracle/_ref) on the same plus random id lists.
Then the library's tokenizer (through tests/cpp/bin/libbpe_host.so, the same tokenizer.cc)
must give the oracle's ids and text, bit for bit, and the reference's where it was built,
and reject what the reference's loader rejects.
"""

from __future__ import annotations

import json
import re
import unicodedata

import pytest

from oracle.bpe import Bpe, byte_alphabet, lossy_utf8, match_at
from tokenizer_helpers import (TOKENIZER_JSON, HostBpe, TokenizerError, cases, random_ids, random_texts,
                               reference_bpe)

GPT2_PATTERN = r"""'s|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+"""


@pytest.fixture(scope="module")
def orc():
    return Bpe(TOKENIZER_JSON)


@pytest.fixture(scope="module")
def hf():
    tokenizers = pytest.importorskip("tokenizers")
    return tokenizers.Tokenizer.from_file(str(TOKENIZER_JSON))


@pytest.fixture(scope="module")
def host():
    h = HostBpe()
    yield h
    h.close()


@pytest.fixture(scope="module")
def ref():
    r = reference_bpe()
    if r is None:
        pytest.skip("oracle/_ref was not built (no reference tree)")
    yield r
    r.close()


def _valid_utf8(data: bytes) -> bool:
    try:
        data.decode("utf-8")
        return True
    except UnicodeDecodeError:
        return False


# ---- pinning the oracle ------------------------------------------------------------------

def test_byte_alphabet_is_gpt2s():
    table = byte_alphabet()
    printable = [b for b in range(256) if table[b] == b]
    assert len(printable) == 188
    assert printable == list(range(0x21, 0x7F)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    moved = [table[b] for b in range(256) if table[b] != b]
    assert moved == list(range(256, 256 + 68))  # in byte order
    assert table[0x20] == 0x120 and table[0x0A] == 0x10A  # 'Ġ' and 'Ċ', GPT-2's space and newline
    tokenizers = pytest.importorskip("tokenizers")
    assert {chr(cp) for cp in table.values()} == set(tokenizers.pre_tokenizers.ByteLevel.alphabet())


@pytest.mark.parametrize("data,want", [
    (b"abc", "abc"),
    ("é中🎉".encode(), "é中🎉"),
    (b"\xe4\xb8", "��"),               # truncated 3-byte sequence: one per byte
    (b"\xc0\x80", "��"),               # overlong NUL
    (b"\xe0\x80\x80", "�" * 3),             # overlong
    (b"\xed\xa0\x80", "�" * 3),             # surrogate U+D800
    (b"\xf4\x90\x80\x80", "�" * 4),         # above U+10FFFF
    (b"\xf8\x88\x80\x80\x80", "�" * 5),     # 5-byte form
    (b"a\x80b", "a�b"),                     # lone continuation byte
    (b"\xf0\x9f\x8e", "�" * 3),             # truncated 4-byte sequence
    (b"\xf4\x8f\xbf\xbf", "\U0010ffff"),         # the last code point
])
def test_lossy_utf8_replaces_each_bad_byte(data, want):
    assert lossy_utf8(data) == want


def _oracle_split(text):
    cps = [ord(c) for c in text]
    out, at = [], 0
    while at < len(cps):
        end = match_at(cps, at, len(cps))
        assert end > at
        out.append(text[at:end])
        at = end
    return out


def test_pattern_split_matches_the_regex():
    regex = pytest.importorskip("regex")
    pat = regex.compile(GPT2_PATTERN)
    texts = random_texts(600, 11, special=False) + ["a  b", "a \n b", "x   ", "  x", "it's", "'sx", "' s", "\t\t"]
    for text in texts:
        assert _oracle_split(text) == pat.findall(text), repr(text)


def _ranges_from_unicodedata(prefix):
    out, start = [], None
    for cp in range(0x110000):
        hit = unicodedata.category(chr(cp)).startswith(prefix)
        if hit and start is None:
            start = cp
        elif not hit and start is not None:
            out.append((start, cp - 1))
            start = None
    if start is not None:
        out.append((start, 0x10FFFF))
    return out


def _ranges_in_inc(name):
    text = (TOKENIZER_JSON.parents[2] / "accelep_amd" / "csrc" / "unicode_ranges.inc").read_text()
    body = text.split(f"constexpr CodeRange {name}[] = {{", 1)[1].split("};", 1)[0]
    return [(int(a, 16), int(b, 16)) for a, b in re.findall(r"\{0x([0-9A-F]+), 0x([0-9A-F]+)\}", body)]


@pytest.fixture(scope="module")
def unicode_tables():
    return {"L": _ranges_from_unicodedata("L"), "N": _ranges_from_unicodedata("N")}


def test_class_tables_match_unicodedata(unicode_tables):
    assert _ranges_in_inc("kLetterRanges") == unicode_tables["L"]
    assert _ranges_in_inc("kNumberRanges") == unicode_tables["N"]


def test_class_tables_match_the_reference(ref, unicode_tables):
    assert ref.unicode_ranges(0) == unicode_tables["L"]
    assert ref.unicode_ranges(1) == unicode_tables["N"]


def test_oracle_matches_tokenizers_on_fixture(orc):
    data = cases()
    for c in data["encode"]:
        assert orc.encode(c["text"]) == c["ids"], repr(c["text"])
        assert orc.decode(c["ids"]) == c["decoded"], repr(c["text"])
    for c in data["decode"]:
        for skip, key in ((True, "skip"), (False, "keep")):
            if _valid_utf8(orc.decode_bytes(c["ids"], skip)):  # `tokenizers` replaces maximal subparts
                assert orc.decode(c["ids"], skip) == c[key], c["ids"]


def test_oracle_matches_tokenizers_on_random_texts(orc, hf):
    for text in random_texts(400, 12):
        ids = hf.encode(text, add_special_tokens=False).ids
        assert orc.encode(text) == ids, repr(text)
        assert orc.decode(ids) == hf.decode(ids, skip_special_tokens=True), repr(text)


def test_oracle_matches_the_reference(orc, ref):
    for text in random_texts(300, 13):
        assert orc.encode(text) == ref.encode(text), repr(text)
    vocab = len(orc.tokens)
    for ids in random_ids(300, 14, vocab) + [[0, 1, 2], []]:
        for skip in (True, False):
            assert orc.decode(ids, skip) == ref.decode(ids, skip), ids


# ---- the library's tokenizer -------------------------------------------------------------

def test_library_matches_oracle_on_fixture(host, orc):
    data = cases()
    assert host.vocab_size() == data["vocab_size"] == len(orc.tokens)
    for c in data["encode"]:
        assert host.encode(c["text"]) == c["ids"], repr(c["text"])
        assert host.decode(c["ids"]) == c["decoded"], repr(c["text"])
    for c in data["decode"]:
        for skip in (True, False):
            assert host.decode(c["ids"], skip) == orc.decode(c["ids"], skip), c["ids"]


def test_library_matches_oracle_on_random_inputs(host, orc):
    for text in random_texts(500, 15):
        assert host.encode(text) == orc.encode(text), repr(text)
    for ids in random_ids(500, 16, len(orc.tokens)):
        for skip in (True, False):
            assert host.decode(ids, skip) == orc.decode(ids, skip), ids


def test_library_matches_the_reference(host, ref):
    texts = random_texts(300, 17) + [c["text"] for c in cases()["encode"]]
    for text in texts:
        assert host.encode(text) == ref.encode(text), repr(text)
    for ids in random_ids(300, 18, host.vocab_size()):
        for skip in (True, False):
            assert host.decode(ids, skip) == ref.decode(ids, skip), ids


def test_long_inputs(host, orc):
    text = "".join(random_texts(40, 19, max_parts=200))
    assert len(text) > 2000
    assert host.encode(text) == orc.encode(text)
    run = "a" * 5000 + " " * 3000 + "7" * 1000
    assert host.encode(run) == orc.encode(run)


def test_errors_match_the_reference(host):
    ref = reference_bpe()
    for bad in (b"\xff", b"ab\xc0\x80", b"\xed\xa0\x80x", b"ok \xe4\xb8"):
        with pytest.raises(TokenizerError, match="prompt is not utf-8"):
            host.encode(bad)
        if ref is not None:
            with pytest.raises(TokenizerError, match="prompt is not utf-8"):
                ref.encode(bad)
    vocab = host.vocab_size()
    for ids in ([vocab], [-1], [0, vocab + 5]):
        with pytest.raises(TokenizerError, match="outside the vocabulary"):
            host.decode(ids)
        if ref is not None:
            with pytest.raises(TokenizerError, match="outside the vocabulary"):
                ref.decode(ids)
    # Bytes outside the vocabulary are dropped: a prompt of them encodes to nothing.
    assert host.encode("\x04\x00") == []
    if ref is not None:
        ref.close()


def test_unloaded_tokenizer_is_an_error():
    h = HostBpe(path=None)
    try:
        with pytest.raises(TokenizerError, match="not loaded"):
            h.encode("a")
        with pytest.raises(TokenizerError, match="not loaded"):
            h.decode([0])
    finally:
        h.close()


def _doc():
    return json.loads(TOKENIZER_JSON.read_text(encoding="utf-8"))


def _mutations():
    def drop(key):
        def f(d):
            del d[key]
        return f

    def setk(path, value):
        def f(d):
            node = d
            for k in path[:-1]:
                node = node[k]
            node[path[-1]] = value
        return f

    def swap_pre(d):
        d["pre_tokenizer"]["pretokenizers"].reverse()

    def vocab_hole(d):
        v = d["model"]["vocab"]
        last = max(v, key=v.get)
        v[last] = v[last] + 5

    def dup_id(d):
        v = d["model"]["vocab"]
        last = max(v, key=v.get)
        v[last] = 3

    def merge_outside(d):
        d["model"]["merges"].append("zzzq qqqz")

    def merge_not_pair(d):
        d["model"]["merges"].append("a b c")

    def added_wrong_id(d):
        d["added_tokens"][0]["id"] = 5

    def added_missing(d):
        d["added_tokens"].append({"id": 3, "content": "<|not in vocab|>", "special": True})

    return {
        "normalizer": setk(["normalizer"], {"type": "NFC"}),
        "no_normalizer_key": drop("normalizer"),
        "post_processor": setk(["post_processor"], {"type": "ByteLevel"}),
        "no_post_processor_key": drop("post_processor"),
        "pre_order": swap_pre,
        "digits_grouped": setk(["pre_tokenizer", "pretokenizers", 0, "individual_digits"], False),
        "prefix_space": setk(["pre_tokenizer", "pretokenizers", 1, "add_prefix_space"], True),
        "no_regex": setk(["pre_tokenizer", "pretokenizers", 1, "use_regex"], False),
        "decoder": setk(["decoder"], {"type": "WordPiece"}),
        "model_type": setk(["model", "type"], "WordPiece"),
        "unk_token": setk(["model", "unk_token"], "a"),
        "dropout": setk(["model", "dropout"], 0.1),
        "byte_fallback": setk(["model", "byte_fallback"], True),
        "fuse_unk": setk(["model", "fuse_unk"], True),
        "suffix": setk(["model", "end_of_word_suffix"], "</w>"),
        "vocab_hole": vocab_hole,
        "duplicate_id": dup_id,
        "merge_outside_vocab": merge_outside,
        "merge_not_a_pair": merge_not_pair,
        "added_wrong_id": added_wrong_id,
        "added_not_in_vocab": added_missing,
        "no_merges": setk(["model", "merges"], []),
    }


@pytest.mark.parametrize("name", sorted(_mutations()))
def test_loader_rejects_what_the_reference_rejects(tmp_path, name):
    doc = _doc()
    _mutations()[name](doc)
    path = tmp_path / "tokenizer.json"
    path.write_text(json.dumps(doc), encoding="utf-8")
    h = HostBpe(path=None)
    try:
        with pytest.raises(TokenizerError):
            h.load(path)
        with pytest.raises(TokenizerError, match="not loaded"):  # a failed load leaves it unloaded
            h.encode("a")
    finally:
        h.close()
    ref = reference_bpe(path=None)
    if ref is not None:
        try:
            with pytest.raises(TokenizerError):
                ref.load(path)
        finally:
            ref.close()


def test_loader_errors_on_unreadable_files(tmp_path):
    h = HostBpe(path=None)
    try:
        with pytest.raises(TokenizerError, match="cannot open"):
            h.load(tmp_path / "missing.json")
        bad = tmp_path / "bad.json"
        bad.write_text('{"model": {"vocab": {"a": 0}', encoding="utf-8")
        with pytest.raises(TokenizerError, match="json"):
            h.load(bad)
        deep = tmp_path / "deep.json"
        deep.write_text('{"model": ' + "[" * 100000 + "]" * 100000 + "}", encoding="utf-8")
        with pytest.raises(TokenizerError, match="nesting too deep"):
            h.load(deep)
    finally:
        h.close()


def test_loader_reads_merges_as_pairs_too(tmp_path, host):
    """Newer `tokenizers` files store merges as [left, right] arrays (the reference reads the
    "left right" strings only); both forms give the same tokenizer here."""
    doc = _doc()
    doc["model"]["merges"] = [m.split(" ") for m in doc["model"]["merges"]]
    path = tmp_path / "pairs.json"
    path.write_text(json.dumps(doc, ensure_ascii=False), encoding="utf-8")
    h = HostBpe(path=path)
    try:
        for text in random_texts(100, 20):
            assert h.encode(text) == host.encode(text)
    finally:
        h.close()


def test_reloading_replaces_the_vocabulary(tmp_path):
    """A second load replaces everything; added-token matching follows the new file."""
    doc = _doc()
    h = HostBpe()
    try:
        before = h.encode("<|im_start|>hi")
        assert before[0] == 1
        doc["added_tokens"] = [a for a in doc["added_tokens"] if a["content"] != "<|im_start|>"]
        path = tmp_path / "fewer.json"
        path.write_text(json.dumps(doc, ensure_ascii=False), encoding="utf-8")
        h.load(path)
        assert h.encode("<|im_start|>hi") == Bpe(path).encode("<|im_start|>hi")
        assert h.encode("<|im_start|>hi")[0] != 1
    finally:
        h.close()
