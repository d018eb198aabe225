"""l3m_encode's ids against fpedd/l3m's own l3m_encode (oracle/_ref, the reference built from its sources,
tokenizer.c:103-170), on vocabularies that merge.

Two vocabularies are trained here by byte-pair counting on a small English text (with digits, contractions
and UTF-8): a SentencePiece-style one (L3M_F_SP_PREFIX: a prefix space, words with their leading space) and
a byte-level BPE one (the GPT-2 pre-tokenizer, L3M_F_DIGITS: digits one by one), each with scores that make
the merge order matter and with duplicate pieces (a lower and an equal score). Each is written into a small
synthetic model file, and both encoders (the backend's host side, l3m_tokenize, needs no GPU) tokenize the
same texts: words, contractions, digit runs, whitespace runs and tabs, punctuation, UTF-8, bytes that are
not UTF-8, an empty text, with and without BOS, and a buffer too small.
"""
import ctypes as C
import struct
from collections import Counter

import pytest

import l3m_amd as A
from oracle.oracle import Reference

SP_PREFIX, DIGITS = 1 << 4, 1 << 5
CORPUS = ("Once upon a time, there was a little girl named Lily. She liked to play outside in the sun. "
          "One day she saw a big red ball near the tree. It's the best ball, she said, and they'd play "
          "with it all day. In 2023 the town had 1250 people; by 2024 it had 1375. We'll see what's next! "
          "The café served crème brûlée and naïve tourists paid 12.50 euros. Über alles: 日本語 テキスト. "
          "Don't stop, won't stop, can't stop. Tom said: \"Hello, world!\" and left at 7:45pm.\n"
          "Tabs\tand  double  spaces   and newlines\n\nare whitespace too.") * 3

TEXTS = [
    "Once upon a time, there was a little girl named Lily.",
    "It's the best ball, she said, and they'd play with it all day.",
    "In 2023 the town had 1250 people; by 2024 it had 1375.",
    "  leading spaces", "trailing spaces   ", "multiple   spaces    between words",
    "Tabs\tand\nnewlines\n\n", "The café served crème brûlée", "日本語 テキスト and Über", "emoji 🚀 rocket",
    "Don't stop, won't stop, can't stop.", "we'll WE'LL 're 've 'm 'll 'd 's 't '", "a", " ", "!!!???...",
    "x1y22z333", "3.14159 and 2,718", "unseenwordsxyz qqq zzz", "Lily Lily Lily ball ball ball",
    "mixed CASE Words And Numbers 42",
]
RAW = [b"bytes \xff\xfe not utf-8 \xc3", b"\xe6\x97\xa5", b"cut \xe6\x97"]


def words(text, sp):
    """Training words: SentencePiece-style words with their leading space, or GPT-2-like runs."""
    if sp:
        return [(" " + w).encode() for w in text.split(" ") if w]
    out, cur = [], b""
    for ch in text.encode():
        c = bytes([ch])
        if cur and (c.isalnum() != cur[-1:].isalnum() or c == b" "):
            out.append(cur)
            cur = b""
        cur += c
    return out + ([cur] if cur else [])


def train(sp, n_merges):
    """Byte-pair merges by frequency: pieces [(bytes, score)], the 256 bytes first."""
    seqs = Counter(tuple(bytes([b]) for b in w) for w in words(CORPUS, sp))
    merges = []
    for rank in range(n_merges):
        pairs = Counter()
        for seq, c in seqs.items():
            for a, b in zip(seq, seq[1:]):
                pairs[(a, b)] += c
        if not pairs:
            break
        (a, b), _ = max(pairs.items(), key=lambda kv: (kv[1], kv[0]))
        merges.append(a + b)
        new = Counter()
        for seq, c in seqs.items():
            out, i = [], 0
            while i < len(seq):
                if i + 1 < len(seq) and seq[i] == a and seq[i + 1] == b:
                    out.append(a + b)
                    i += 2
                else:
                    out.append(seq[i])
                    i += 1
            new[tuple(out)] += c
        seqs = new
    pieces = [(bytes([i]), -1e9) for i in range(256)]
    # SentencePiece-style scores grow with frequency; byte-level BPE uses -rank (both: earlier merges first)
    pieces += [(m, (1000.0 - r) if sp else float(-r)) for r, m in enumerate(merges)]
    # duplicates: one with a lower score (never chosen), one with an equal score (the lower id is chosen)
    pieces += [(merges[3], pieces[256 + 3][1] - 5.0), (merges[7], pieces[256 + 7][1])]
    return pieces


def write_vocab_model(path, pieces, flags):
    """A tiny synthetic model whose tokenizer section holds these pieces (vocab = their count + BOS, EOS)."""
    n = len(pieces) + 2
    cfg = A.Config("tok", dim=64, n_layers=1, n_heads=2, n_kv_heads=2, ffn_dim=64, vocab=n, ctx=32, dtype="f32")
    A.write_model(path, cfg)
    raw = bytearray(path.read_bytes())
    tok_off, = struct.unpack_from("<Q", raw, 80)
    max_len = max(len(b) for b, _ in pieces)
    sec = bytearray(struct.pack("<IiiI", n, n - 2, n - 1, max_len))
    for b, s in pieces + [(b"", 0.0), (b"", 0.0)]:
        sec += struct.pack("<fH", s, len(b)) + b
    struct.pack_into("<I", raw, 24, struct.unpack_from("<I", raw, 24)[0] | flags)
    path.write_bytes(bytes(raw[:tok_off]) + bytes(sec))
    return path


def ours(path, text, bos, cap):
    out = (C.c_int32 * cap)()
    n = A.lib().l3m_tokenize(str(path).encode(), text, int(bos), out, cap)
    return None if n < 0 else list(out[:n])


def theirs(model, text, bos, cap):
    out = (C.c_int32 * cap)()
    n = model.r.lib.l3m_encode(model.h, text, int(bos), out, cap)
    return None if n < 0 else list(out[:n])


@pytest.fixture(scope="module")
def reference():
    if not Reference.available():
        pytest.skip("oracle/_ref (the reference built from source) is not present")
    return Reference()


@pytest.mark.parametrize("style", ["sentencepiece", "bytelevel"])
def test_encode_matches_reference(reference, tmp_path, style):
    sp = style == "sentencepiece"
    pieces = train(sp, 160)
    assert max(len(b) for b, _ in pieces) >= 4
    path = write_vocab_model(tmp_path / f"{style}.l3m", pieces, SP_PREFIX if sp else DIGITS)
    model = reference.load(path)
    merged = 0
    for text in [t.encode() for t in TEXTS] + RAW + [b""]:
        for bos in (True, False):
            want = theirs(model, text, bos, 4 * len(text) + 8)
            got = ours(path, text, bos, 4 * len(text) + 8)
            assert got == want, (style, text, bos, got, want)
            merged += sum(i >= 256 for i in want)
    assert merged > 50                                # the merges are exercised, not just the bytes
    # a buffer too small: -1 exactly where the reference gives -1 (the unmerged ids of a piece must fit too)
    text = TEXTS[0].encode()
    fits = [cap for cap in range(1, 80) if theirs(model, text, True, cap) is not None]
    assert fits and ours(path, text, True, fits[0]) == theirs(model, text, True, fits[0])
    assert ours(path, text, True, fits[0] - 1) is None


def test_byte_vocabulary_encodes_bytes(reference, tmp_path):
    """The synthetic models' vocabulary (256 byte pieces, then empty ones; max_len 1): one id per byte."""
    cfg = A.Config("bytes", dim=64, n_layers=1, n_heads=2, n_kv_heads=2, ffn_dim=64, vocab=300, ctx=32, dtype="f32")
    path = A.write_model(tmp_path / "bytes.l3m", cfg)
    model = reference.load(path)
    for text in [t.encode() for t in TEXTS[:6]] + RAW:
        assert ours(path, text, False, 256) == theirs(model, text, False, 256) == list(text)
