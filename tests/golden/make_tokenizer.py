"""Writes the tokenizer fixtures: a small tokenizer.json in the SmolLM2 form and the expected
encode/decode of a list of strings.

    python3 tests/golden/make_tokenizer.py

* tokenizer_small.json: a byte-level BPE trained with Hugging Face `tokenizers` (0.22.2 here)
  on a synthetic corpus, with SmolLM2-135M's pipeline (model BPE; normalizer and
  post-processor null; pre-tokenizer Digits(individual_digits) then ByteLevel(no prefix
  space, regex); ByteLevel decoder; special tokens <|endoftext|>, <|im_start|>, <|im_end|>
  first). As in SmolLM2's vocabulary (AccelEP README.md:43), 21 of GPT-2's 256 byte symbols
  are not in the vocabulary (bytes 0x00-0x08 and 0x0E-0x19): encode drops them. Merges are
  written as "left right" strings, the form AccelEP's loader reads (src/bpe.cc:806-823).
* tokenizer_cases.json: for each string (the 24 samples of AccelEP tests/test_serve.py:192-221
  and more), the ids `tokenizers` gives (encode without special-token insertion) and its
  decode of those ids with skip_special_tokens; plus decode-only id lists (special tokens,
  ids that split a UTF-8 sequence).

The expected values come from `tokenizers`, which AccelEP's own tokenizer test uses as the
truth (tests/test_serve.py:182-234).
"""

from __future__ import annotations

import json
import random
from pathlib import Path

from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers

HERE = Path(__file__).resolve().parent
SPECIAL = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
MISSING_BYTES = list(range(0x00, 0x09)) + list(range(0x0E, 0x1A))
VOCAB = 1400

WORDS = """the of and to in is was for on that with as by at from his her it an were are which this be
has had or not but also have one their its first new after two who they more been other she he when
time there into during all would about over only up out world city year state school some world
people can may later most made such between used called many where then these under three however
world during known part while both because around music team film before until through second
capital france paris germany berlin europe river mountain language history science number small
large quick brown fox jumps lazy dog hello friend today tomorrow yesterday model token merge byte
device kernel memory stream graph wave tile shard stripe page buffer queue vector matrix""".split()
UNICODE = ["café", "naïve", "façade", "Ελληνικά", "русский", "язык", "中文", "日本語", "한국어", "עברית",
           "العربية", "हिन्दी", "ไทย", "Ωmega", "Straße", "Ærø", "😀", "🎉", "👍🏽", "∑", "√2", "½", "Ⅻ", "٣",
           "०१२", "①②", "²³", "—", "…", "«", "»", "€", "£", "¥"]
PUNCT = [".", ",", "!", "?", ";", ":", "'", '"', "(", ")", "-", "--", "/", "#", "@", "&", "*", "...", "!?"]
CONTRACTIONS = ["'s", "'t", "'re", "'ve", "'m", "'ll", "'d", "'S", "'T"]
SPACES = [" ", " ", " ", " ", "  ", "   ", "\n", "\n\n", "\t", " \n", " ", "　", "\r\n"]


def corpus(lines: int, seed: int):
    r = random.Random(seed)
    for _ in range(lines):
        parts = []
        for _ in range(r.randint(4, 24)):
            pick = r.random()
            if pick < 0.62:
                w = r.choice(WORDS)
                parts.append(w.capitalize() if r.random() < 0.15 else w)
            elif pick < 0.72:
                parts.append(str(r.randint(0, 10 ** r.randint(1, 6))))
            elif pick < 0.80:
                parts.append(r.choice(UNICODE))
            elif pick < 0.92:
                parts.append(r.choice(PUNCT))
            else:
                parts.append(r.choice(WORDS) + r.choice(CONTRACTIONS))
            parts.append(r.choice(SPACES))
        yield "".join(parts)


def build_tokenizer() -> dict:
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Digits(individual_digits=True),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=True),
    ])
    tok.decoder = decoders.ByteLevel()
    byte_alphabet = pre_tokenizers.ByteLevel.alphabet()
    mapping = _byte_symbols()
    dropped = {mapping[b] for b in MISSING_BYTES}
    alphabet = sorted(ch for ch in byte_alphabet if ch not in dropped)
    trainer = trainers.BpeTrainer(vocab_size=VOCAB, special_tokens=SPECIAL, initial_alphabet=alphabet,
                                  show_progress=False)
    tok.train_from_iterator(corpus(6000, 20261202), trainer=trainer)
    doc = json.loads(tok.to_str())
    doc["normalizer"] = None
    doc["post_processor"] = None
    # The loader of AccelEP reads merges as "left right" strings; byte-level tokens never
    # contain a space, so the two forms hold the same pairs.
    doc["model"]["merges"] = [m if isinstance(m, str) else f"{m[0]} {m[1]}" for m in doc["model"]["merges"]]
    vocab = doc["model"]["vocab"]
    assert not any(sym in vocab for sym in dropped), "a dropped byte symbol came back from the corpus"
    assert sorted(vocab.values()) == list(range(len(vocab)))
    return doc


def _byte_symbols():
    """GPT-2's byte -> symbol table (printable bytes stand for themselves, the rest take
    U+0100.. in byte order)."""
    keep = list(range(0x21, 0x7F)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    out = {}
    extra = 0
    for b in range(256):
        if b in keep:
            out[b] = chr(b)
        else:
            out[b] = chr(256 + extra)
            extra += 1
    return out


def samples():
    # AccelEP tests/test_serve.py:192-221.
    ref = [
        "", "Hello", "Hey 123 friend!", "dog's day\nnext", "café", "🎉", "a  b", "a\tb", "\x04", "a\x04b", "!\x04!",
        ".\x04.", "\n\x04\n", " \x04!", " \x04 ", "\x00", "\x1f ", "hello\x04", "\U00040000", "A\U00040000B",
        "!\U00040000@", "<|im_start|>hi<|im_end|>", "The capital of France is",
        ("<|im_start|>system\nYou are a helpful AI assistant named SmolLM, trained by Hugging Face<|im_end|>\n"
         "<|im_start|>user\nThe capital of France is<|im_end|>\n<|im_start|>assistant\n"),
    ]
    more = [
        " ", "  ", "\n", "   \n", "a ", "a  ", "a   b", " a", "  a", "\t\t x", "x \t", "x  y", "　　z",
        "it's", "IT'S", "we're they've I'll he'd I'm don't", "'s's'", "'", "''", "' s", "rock'n'roll",
        "12345", "3.14159", "1,000,000", "x1y22z333", "٣٤٥ and ①② and ²³ and Ⅻ", "½ + ¼", "v2.0-rc1",
        "Ελληνικά русский 中文 日本語 한국어", "naïve façade Straße", "עברית العربية हिन्दी ไทย",
        "😀😀 👍🏽 🎉!", "a😀b", "é", "tab\there", "line1\r\nline2", "\x1b[0m", "\x7f\x80",
        "<|endoftext|>", "<|im_end|><|im_end|>", "<|im_start", "<|im_start|", "x<|endoftext|>y",
        "<|im_start|><|endoftext|>", "hello world " * 8, "The quick brown fox jumps over the lazy dog.",
        "Paris is the capital of France; Berlin, of Germany!", "memory -- stream ... graph?!",
        "  leading and trailing  ", "\n\n\nparagraph\n\n", "mixed sep x", "\u0085nel",
        "ab\x00cd", "\x00\x00", "\x19\x1a\x1b",
    ]
    return ref + more


def decode_only(tok: Tokenizer, vocab_size: int):
    r = random.Random(7)
    cases = [[0], [1, 2], [0, 1, 2], list(range(0, 40)), [vocab_size - 1, vocab_size - 2]]
    cases += [[r.randrange(vocab_size) for _ in range(r.randint(1, 30))] for _ in range(40)]
    # Ids that split multi-byte characters: the bytes of "é" and "🎉" one at a time.
    for text in ["é", "🎉", "中"]:
        ids = []
        for b in text.encode("utf-8"):
            sym = _byte_symbols()[b]
            if tok.token_to_id(sym) is not None:
                ids.append(tok.token_to_id(sym))
        cases.append(ids)
        cases.append(ids[:-1])
        cases.append(ids[1:])
    out = []
    for ids in cases:
        out.append(dict(ids=ids, keep=tok.decode(ids, skip_special_tokens=False),
                        skip=tok.decode(ids, skip_special_tokens=True)))
    return out


def main():
    doc = build_tokenizer()
    path = HERE / "tokenizer_small.json"
    path.write_text(json.dumps(doc, ensure_ascii=False, indent=1) + "\n", encoding="utf-8")
    tok = Tokenizer.from_file(str(path))
    cases = []
    for text in samples():
        ids = tok.encode(text, add_special_tokens=False).ids
        cases.append(dict(text=text, ids=ids, decoded=tok.decode(ids, skip_special_tokens=True)))
    out = dict(tokenizers_version=__import__("tokenizers").__version__, vocab_size=tok.get_vocab_size(),
               encode=cases, decode=decode_only(tok, tok.get_vocab_size()))
    (HERE / "tokenizer_cases.json").write_text(json.dumps(out, ensure_ascii=False, indent=1) + "\n", encoding="utf-8")
    print(f"wrote {path.name} ({tok.get_vocab_size()} tokens) and tokenizer_cases.json ({len(cases)} strings)")


if __name__ == "__main__":
    main()
