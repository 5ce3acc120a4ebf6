"""Writes the tokenizer fixtures under tests/golden/tok/.

Two synthetic vocabulary files in the reference's formats (the llama2.c
format LLamaTokenizer reads: int32 max piece length, then per piece a float
score, an int32 length and the bytes; and the format Gpt2Tokenizer reads:
per word a uint32 length and the bytes), made here from a fixed recipe, and
the token ids and decoded pieces the reference's own tokenizers
(gten/tokenizer.cpp, compiled into oracle/_ref) produce for them.  Runs in
the build container only; the tests read the files it writes.

    python tests/golden/make_tok_golden.py
"""
import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "tok")
sys.path.insert(0, os.path.join(os.path.dirname(HERE)))
import oracle_lib as OL  # noqa: E402

# texts both tokenizers see (bytes: some are not valid UTF-8)
TEXTS = [
    b"", b" ", b"Hello, world!", b"hello world hello", b"the cat sat on the mat.", b"  leading and  double spaces",
    b"tabs\tand\nnewlines\r\n", b"numbers 12345 and 3.14159", "café naïve résumé".encode(),
    "中文测试：你好".encode(), "emoji \U0001F600\U0001F389 ∑∫".encode(),
    b"it's we're they've I'm you'll he'd 'quoted'", b"\xff\xfe bad \xc3 bytes", b"\xf0\x9f\x98\x80\x80\x80 five",
    b"def f(x):\n    return x**2  # comment", b"aaaaaaaaaaaaaaaa", b"abababababab abab", b"<0x41> looks like a byte",
    b"the the the then there their", b"   ",
]


def bpe_vocab():
    """(pieces, scores): <unk> <s> </s>, the 256 byte pieces, single
    characters, then substrings of a sample text with scores drawn to one
    decimal (so some tie), a duplicated piece and a piece scored below
    -1e10."""
    pieces = [b"<unk>", b"<s>", b"</s>"] + [f"<0x{i:02X}>".encode() for i in range(256)]
    scores = [0.0] * len(pieces)
    singles = [bytes([c]) for c in range(32, 127)] + ["é".encode(), "中".encode(), b"\t", b"\n"]
    for s in singles:
        pieces.append(s)
        scores.append(-100.0)
    rng = np.random.default_rng(2024)
    sample = b" the cat sat on the mat hello world hello there their then caf abab aaaa return def"
    words = set()
    for w in sample.split(b" "):
        w = b" " + w
        for a in range(len(w)):
            for b in range(a + 2, min(len(w), a + 6) + 1):
                words.add(w[a:b])
    for w in sorted(words):
        pieces.append(w)
        scores.append(float(np.round(rng.normal(-5.0, 3.0), 1)))  # one decimal: ties happen
    pieces.append(b" the")  # a duplicate piece (both ids exist; lookups resolve to one)
    scores.append(5.0)
    pieces.append(b"xyz")
    scores.append(-2e10)  # below the merge loop's -1e10 floor: never merged
    pieces += [b"x", b"y", b"z"]
    scores += [-1.0, -1.0, -1.0]
    return pieces, scores


def words_vocab():
    words = [bytes([c]) for c in range(32, 127)] + [b"\n", b"\t", b"\r", "é".encode()]
    words += [b"Hello", b" world", b" hello", b"hello", b" the", b" cat", b"the", b" mat", b"'s", b"'re", b"'ve",
              b" 123", b"45", b" 3", b".14", b"  ", b"   ", b" sat", b" on", b" caf", b" bad", b" bytes", b" return",
              b"def", b" f", b"(x", b"):", b"**", b" comment", b"aaaa", b"abab", b" abab", b" the"]  # " the" twice
    words += ["中".encode(), "文".encode(), b"\xf0\x9f\x98\x80"]
    return words


def write_bpe(path, pieces, scores):
    with open(path, "wb") as f:
        f.write(struct.pack("<i", max(len(p) for p in pieces)))
        for p, s in zip(pieces, scores):
            f.write(struct.pack("<fi", s, len(p)) + p)


def write_words(path, words):
    with open(path, "wb") as f:
        for w in words:
            f.write(struct.pack("<I", len(w)) + w)


# (name, kind, file, vocab size, eos, prompt prefix, prompt suffix, token prefix, token suffix)
CONFIGS = [
    ("bpe_plain", "bpe", "bpe_vocab.bin", None, 2, "", "", [], []),
    ("bpe_chat", "bpe", "bpe_vocab.bin", None, 2, "user\n", "", [1, 5], [6, 7, 8]),
    # Gpt2Tokenizer hard-codes Zephyr's chat prefix and suffix (tokenizer.h:59-60)
    ("words", "words", "words_vocab.bin", None, 0, "", "", [27, 91, 882, 91, 29, 397],
     [100257, 198, 27, 91, 78191, 91, 397]),
]


def main():
    os.makedirs(OUT, exist_ok=True)
    pieces, scores = bpe_vocab()
    write_bpe(os.path.join(OUT, "bpe_vocab.bin"), pieces, scores)
    words = words_vocab()
    write_words(os.path.join(OUT, "words_vocab.bin"), words)
    ref = OL.Reference()
    fx = {}
    for name, kind, fname, _, eos, pp, ps, tp, ts in CONFIGS:
        path = os.path.join(OUT, fname).encode()
        n = len(pieces) if kind == "bpe" else len(words)
        tp_a, ts_a = np.array(tp, np.int32), np.array(ts, np.int32)
        if kind == "bpe":
            h = ref.tok_llama_create(path, n, eos, pp.encode(), ps.encode(), OL.ptr(tp_a), len(tp), OL.ptr(ts_a),
                                     len(ts))
        else:
            h = ref.tok_gpt2_create(path, n, eos)
        enc = []
        for t in TEXTS:
            buf = np.zeros(4096, np.int32)
            cnt = ref.tok_encode(h, t, OL.ptr(buf), 4096)
            enc.append(buf[:cnt].tolist())
        dec = {str(prev): [ref.tok_decode(h, prev, i).hex() for i in range(n + 2)] for prev in (1, 9)}
        ref.tok_free(h)
        fx[name] = dict(kind=kind, file=fname, vocab_size=n, eos=eos, prompt_prefix=pp, prompt_suffix=ps,
                        tokens_prefix=tp, tokens_suffix=ts, encode=enc, decode=dec)
    fx["texts"] = [t.hex() for t in TEXTS]
    with open(os.path.join(OUT, "expected.json"), "w") as f:
        json.dump(fx, f)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
