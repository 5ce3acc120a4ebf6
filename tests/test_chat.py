"""The text path: prompt text -> tokenizer -> model -> tokens -> text, as
the reference's greedy_sample and topk_sample (src/gten/sampler.cpp:11-143)
run it behind nanochat.cpp's chat loop.

* Fixture (tests/golden/chat.json, written by make_chat_golden.py): the text
  the reference's own greedy_sample writes for three prompts on small
  synthetic models of the four architectures, through the reference's
  LLamaTokenizer over the synthetic vocabulary of tests/golden/tok/ with chat
  prefixes and suffixes; and the sampled text of the reference harness's
  mt19937 stream decoded the way topk_sample decodes it.
* CPU: the fixture is pinned twice -- the reference build reproduces it, and
  the oracle's greedy stream decoded by this package's tokenizer gives the
  same text.
* GPU: nc_greedy_sample / nc_topk_sample give the fixture's text byte for
  byte, the streamed pieces add up to it, and errors are reported.
"""
import json
import os

import numpy as np
import pytest

import oracle_lib as OL
from nc_pkg import nc
from workloads import CHAT, CHAT_TOPK, config_of

HERE = os.path.dirname(os.path.abspath(__file__))
TOK = os.path.join(HERE, "golden", "tok")


def fixture():
    with open(os.path.join(HERE, "golden", "chat.json")) as f:
        return json.load(f)


def tok_config():
    with open(os.path.join(TOK, "expected.json")) as f:
        return json.load(f)[fixture()["tokenizer"]]


def product_tokenizer():
    c = tok_config()
    return nc.Tokenizer.bpe(os.path.join(TOK, c["file"]), c["vocab_size"], c["eos"], c["prompt_prefix"],
                            c["prompt_suffix"], c["tokens_prefix"], c["tokens_suffix"])


def test_fixture_covers_every_chat_model():
    fx = fixture()
    assert sorted(fx["models"]) == sorted(CHAT)
    assert fx["topk"] == CHAT_TOPK
    # the texts are the reference's: every one ends with greedy_sample's "\n"
    for runs in fx["models"].values():
        for r in runs:
            assert bytes.fromhex(r["text_hex"]).endswith(b"\n")
            assert bytes.fromhex(r["topk_text_hex"]).endswith(b"\n")


@pytest.mark.parametrize("name", list(CHAT))
def test_reference_reproduces_fixture(reference, name):
    c = tok_config()
    tp, ts = np.array(c["tokens_prefix"], np.int32), np.array(c["tokens_suffix"], np.int32)
    tok = reference.tok_llama_create(os.path.join(TOK, c["file"]).encode(), c["vocab_size"], c["eos"],
                                     c["prompt_prefix"].encode(), c["prompt_suffix"].encode(), OL.ptr(tp), len(tp),
                                     OL.ptr(ts), len(ts))
    cfg = config_of(CHAT[name])
    m = reference.model_create(cfg, CHAT[name]["seed"])
    try:
        for r in fixture()["models"][name]:
            got = reference.greedy_sample_text(m, tok, r["prompt"].encode(), cfg.max_ctx, cfg.max_ctx)
            assert got.hex() == r["text_hex"], r["prompt"]
    finally:
        reference.model_free(m)
        reference.tok_free(tok)


@pytest.mark.parametrize("name", list(CHAT))
def test_oracle_stream_decodes_to_fixture(oracle, name):
    """The oracle's greedy stream for the tokenized prompt, decoded with this
    package's (host) tokenizer by greedy_sample's rule, is the fixture text."""
    w = CHAT[name]
    cfg = config_of(w)
    m = oracle.model_create(cfg, w["seed"])
    t = product_tokenizer()
    try:
        for r in fixture()["models"][name]:
            ids = t.encode(r["prompt"].encode())
            n_gen = cfg.max_ctx - len(ids)
            out = np.zeros(max(n_gen, 1), np.int32)
            got = oracle.generate_greedy(m, OL.ptr(ids), len(ids), n_gen, OL.ptr(out)) if n_gen > 0 else 0
            text, prev = b"", 1
            for tok in out[:got].tolist():
                if tok == t.eos:
                    break
                text += t.decode(prev, tok)
                prev = tok
            assert (text + b"\n").hex() == r["text_hex"], r["prompt"]
    finally:
        oracle.model_free(m)
        t.close()


def gpu_model(gpu, name):
    w = CHAT[name]
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig))
    m.init_synthetic(w["seed"])
    return m


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CHAT))
def test_greedy_sample_text_matches_reference(gpu, name):
    m = gpu_model(gpu, name)
    t = product_tokenizer()
    try:
        for r in fixture()["models"][name]:
            pieces = []
            text, n = gpu.greedy_sample(m, t, r["prompt"], on_text=pieces.append)
            assert text.hex() == r["text_hex"], (name, r["prompt"])
            assert b"".join(pieces) == text
            # one piece per token, then the closing newline
            assert len(pieces) == n + 1
    finally:
        m.close()
        t.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CHAT))
def test_topk_sample_text_matches_reference(gpu, name):
    m = gpu_model(gpu, name)
    t = product_tokenizer()
    k = CHAT_TOPK
    try:
        for r in fixture()["models"][name]:
            text, _ = gpu.topk_sample(m, t, r["prompt"], temp=k["temp"], top_k=k["top_k"], seed=k["seed"])
            assert text.hex() == r["topk_text_hex"], (name, r["prompt"])
    finally:
        m.close()
        t.close()


@pytest.mark.gpu
def test_sample_text_limits(gpu):
    name = "chat-llama-q8"
    m = gpu_model(gpu, name)
    t = product_tokenizer()
    try:
        full = fixture()["models"][name][0]
        want = bytes.fromhex(full["text_hex"])
        n_prompt = len(t.encode(full["prompt"].encode()))
        # a shorter n_predict: the same text cut after n_predict - prompt tokens
        text, n = gpu.greedy_sample(m, t, full["prompt"], n_predict=n_prompt + 5)
        assert n <= 5 and want.startswith(text[:-1]) and text.endswith(b"\n")
        # no room to generate: only the newline, as the reference prints it
        assert gpu.greedy_sample(m, t, full["prompt"], n_predict=n_prompt) == (b"\n", 0)
        with pytest.raises(gpu.HipError, match="max_ctx"):
            gpu.greedy_sample(m, t, full["prompt"], n_predict=m.cfg.max_ctx + 1)
        # the model is reusable after every call: the full text again
        assert gpu.greedy_sample(m, t, full["prompt"])[0] == want
    finally:
        m.close()
        t.close()


def test_chat_program_arguments():
    """The chat program (built next to the library) checks its arguments as
    nanochat.cpp does before touching a device."""
    import subprocess
    exe = os.path.join(os.path.dirname(nc.LIB_PATH), "nanochat")
    if not os.path.exists(exe):
        pytest.fail(f"{exe} is missing: run __graft_entry__.build()")
    r = subprocess.run([exe, "--help"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "MODEL_NAME" in r.stdout
    r = subprocess.run([exe, "-m", "gpt9"], capture_output=True, text=True, timeout=60)
    assert r.returncode != 0 and "Unknown or missing model name" in r.stderr
    r = subprocess.run([exe, "-m", "tinyllama", "--npred", "0"], capture_output=True, text=True, timeout=60)
    assert r.returncode != 0 and "npred" in r.stderr
    r = subprocess.run([exe, "-m", "tinyllama", "--temp", "-1"], capture_output=True, text=True, timeout=60)
    assert r.returncode != 0 and "temp" in r.stderr
