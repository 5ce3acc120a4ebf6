"""Writes tests/golden/chat.json: the text the reference's own greedy_sample
(src/gten/sampler.cpp:11-60) writes for a prompt, driving small synthetic
models of each architecture through the reference's LLamaTokenizer
(src/gten/tokenizer.cpp) over the synthetic vocabulary of tests/golden/tok/
(bpe_vocab.bin, with the chat prefixes and suffixes of the "bpe_chat"
fixture, as nanochat.cpp:189-229 builds a tokenizer).  Sampled text: the
harness's topk stream with std::mt19937(seed), decoded with the reference's
tokenizer as topk_sample (sampler.cpp:78-138) decodes it.

Runs in the build container only (it needs oracle/_ref/libgten_ref.so, the
reference's sources compiled by oracle/Makefile, sampler.cpp included).

    python tests/golden/make_chat_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import oracle_lib as OL  # noqa: E402
from workloads import CHAT, CHAT_PROMPTS, CHAT_TOKENIZER, CHAT_TOPK, config_of  # noqa: E402


def tokenizer(ref):
    with open(os.path.join(HERE, "tok", "expected.json")) as f:
        c = json.load(f)[CHAT_TOKENIZER]
    tp = np.array(c["tokens_prefix"], np.int32)
    ts = np.array(c["tokens_suffix"], np.int32)
    path = os.path.join(HERE, "tok", c["file"]).encode()
    return ref.tok_llama_create(path, c["vocab_size"], c["eos"], c["prompt_prefix"].encode(),
                                c["prompt_suffix"].encode(), OL.ptr(tp), len(tp), OL.ptr(ts), len(ts))


def main():
    ref = OL.Reference()
    tok = tokenizer(ref)
    out = {"tokenizer": CHAT_TOKENIZER, "topk": CHAT_TOPK, "models": {}}
    for name, w in CHAT.items():
        cfg = config_of(w)
        m = ref.model_create(cfg, w["seed"])
        runs = []
        for prompt in CHAT_PROMPTS:
            text = ref.greedy_sample_text(m, tok, prompt.encode(), cfg.max_ctx, cfg.max_ctx)
            # topk_sample's text loop (sampler.cpp:78-138) over the harness's
            # sampled stream with std::mt19937(seed) (the reference seeds it
            # from std::random_device)
            ids = np.zeros(4096, np.int32)
            n_p = ref.tok_encode(tok, prompt.encode(), OL.ptr(ids), len(ids))
            n_gen = cfg.max_ctx - n_p
            gen = np.zeros(max(n_gen, 1), np.int32)
            got = ref.generate_topk(m, OL.ptr(ids), n_p, n_gen, CHAT_TOPK["temp"], CHAT_TOPK["top_k"],
                                    CHAT_TOPK["seed"], OL.ptr(gen)) if n_gen > 0 else 0
            pieces, prev = [], 1
            for t in gen[:got].tolist():
                pieces.append(ref.tok_decode(tok, prev, t) or b"")
                prev = t
            topk_text = b"".join(pieces) + b"\n"
            runs.append({"prompt": prompt, "text_hex": text.hex(), "topk_text_hex": topk_text.hex()})
            print(name, repr(prompt), repr(text[:80]), len(text), repr(topk_text[:60]), len(topk_text))
        out["models"][name] = runs
        ref.model_free(m)
    ref.tok_free(tok)
    with open(os.path.join(HERE, "chat.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
