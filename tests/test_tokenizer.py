"""The tokenizers (gten/tokenizer.cpp) in front of and behind the decode
path: nc_tokenizer_* against the reference's LLamaTokenizer and
Gpt2Tokenizer.

* Fixtures (tests/golden/tok/, written by make_tok_golden.py with the
  reference's tokenizers): two synthetic vocabularies in the reference's file
  formats, with merges that tie, a duplicated piece, a piece scored below the
  merge floor and byte fallback; token ids of 20 texts (invalid UTF-8, a
  5-byte sequence, CJK, emoji, whitespace runs) and every decoded piece.
* The real vocabularies of nanochat.cpp's models (read from the reference
  tree where it exists): the product's tokenizer for each model against the
  reference's, built as nanochat.cpp:189-229 builds it, on the same texts
  plus longer and random ones, and every id decoded.
"""
import json
import os

import numpy as np
import pytest

import oracle_lib as OL
from nc_pkg import nc

TOK = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tok")


def fixtures():
    with open(os.path.join(TOK, "expected.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("name", ["bpe_plain", "bpe_chat", "words"])
def test_tokenizer_matches_reference_fixtures(name):
    fx = fixtures()
    c = fx[name]
    path = os.path.join(TOK, c["file"])
    if c["kind"] == "bpe":
        t = nc.Tokenizer.bpe(path, c["vocab_size"], c["eos"], c["prompt_prefix"], c["prompt_suffix"],
                             c["tokens_prefix"], c["tokens_suffix"])
    else:
        t = nc.Tokenizer.words(path, c["vocab_size"], c["eos"], c["tokens_prefix"], c["tokens_suffix"])
    texts = [bytes.fromhex(h) for h in fx["texts"]]
    for text, want in zip(texts, c["encode"]):
        assert t.encode(text).tolist() == want, text
    for prev, pieces in c["decode"].items():
        got = [t.decode(int(prev), i).hex() for i in range(len(pieces))]
        assert got == pieces, prev
    assert t.eos == c["eos"]
    t.close()


def test_tokenizer_errors():
    with pytest.raises(nc.HipError, match="cannot open"):
        nc.Tokenizer.bpe(os.path.join(TOK, "absent.bin"), 10, 2)
    with pytest.raises(nc.HipError, match="ends"):  # more pieces asked for than the file holds
        nc.Tokenizer.bpe(os.path.join(TOK, "bpe_vocab.bin"), 100000, 2)
    with pytest.raises(nc.HipError, match="unknown model"):
        nc.Tokenizer.for_model("gpt9", os.path.join(TOK, "bpe_vocab.bin"))


# nanochat.cpp:189-229: vocabulary file, then the reference tokenizer's constructor arguments
MODELS = {
    "tinyllama": ("tinyllama_tokenizer.bin", "llama", (32000, 32002, b"user\n", b"", [1, 32001],
                                                       [32002, 29871, 13, 32001, 20255, 13])),
    "minicpm": ("minicpm_tokenizer.bin", "llama", (122753, 2, "<用户>".encode(), "<AI>".encode(), [], [])),
    "openelm_sm": ("tinyllama_tokenizer.bin", "llama", (32000, 32002, b"", b"", [1], [])),
    "zephyr": ("zephyr_tokenizer.bin", "gpt2", (100352, 100257)),
}


def more_texts():
    rng = np.random.default_rng(11)
    para = ("The quick brown fox jumps over the lazy dog. It's 3.14 o'clock; we've 42 apples. "
            "机器学习是人工智能的一个分支。Ünïcödé tëxt ñ 😀\n\t  end").encode()
    out = [para, para * 4]
    for _ in range(6):  # random printable ASCII and random bytes (no NUL)
        out.append(bytes(rng.integers(32, 127, 60).tolist()))
        out.append(bytes(rng.integers(1, 256, 40).tolist()))
    return out


@pytest.mark.parametrize("model", list(MODELS))
def test_tokenizer_matches_reference_on_real_vocabularies(reference, model):
    fname, kind, args = MODELS[model]
    path = os.path.join(OL.REFERENCE_ROOT, "assets", "tokenizers", fname)
    if not os.path.exists(path):
        pytest.skip("the reference's vocabulary files are not here")
    if kind == "llama":
        n, eos, pp, ps, tp, ts = args
        tp_a, ts_a = np.array(tp, np.int32), np.array(ts, np.int32)
        h = reference.tok_llama_create(path.encode(), n, eos, pp, ps, OL.ptr(tp_a), len(tp), OL.ptr(ts_a), len(ts))
    else:
        n, eos = args
        h = reference.tok_gpt2_create(path.encode(), n, eos)
    t = nc.Tokenizer.for_model(model, path)
    try:
        fx = fixtures()
        texts = [bytes.fromhex(x) for x in fx["texts"]] + more_texts()
        buf = np.zeros(1 << 15, np.int32)
        for text in texts:
            cnt = reference.tok_encode(h, text, OL.ptr(buf), len(buf))
            assert t.encode(text).tolist() == buf[:cnt].tolist(), text
        ids = range(n + 2) if n <= 40000 else list(range(0, n + 2, 7)) + list(range(n - 500, n + 2))
        for prev in (1, 9):
            for i in ids:
                assert t.decode(prev, i) == (reference.tok_decode(h, prev, i) or b""), (prev, i)
        assert t.eos == eos
    finally:
        reference.tok_free(h)
        t.close()
