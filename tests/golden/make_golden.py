"""Writes the golden fixtures under tests/golden/ from the reference's own code.

Runs in the build container only (it needs oracle/_ref/libgten_ref.so, the
reference's gten sources compiled by oracle/Makefile).  For every workload it
builds the model from the reference's modules with the synthetic weights and
runs greedy_sample's loop (src/gten/sampler.cpp:17-48) over the reference's
Model::logits: the prompt with start_pos = 0, then each decode step with
start_pos = n - 1 (the reference's K/V caches carry the earlier rows).  It
records the prompt, the generated tokens, digests of the prefill logits and
of every layer's residual-stream row, the top prefill logits, and at decode
steps 1, 2, 16, 64 and the last one the digests of that step's fp32 logits
and of every layer's row at its position.  Small models of every
architecture are recorded the same way, with their full prefill logits.

    python tests/golden/make_golden.py [workload ...]
    python tests/golden/make_golden.py --topk [workload ...]   (sampled streams)
"""
import hashlib
import json
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import gten_file as G  # noqa: E402
import oracle_lib as OL  # noqa: E402
from workloads import LONG, SMALL, WIDE, config_of, prompt_of  # noqa: E402
from nc_pkg import nc  # noqa: E402

# decode steps (1 = the first step after the prompt) whose digests are kept
DIGEST_STEPS = (1, 2, 16, 64)


def sha(b):
    return hashlib.sha256(np.ascontiguousarray(b).tobytes()).hexdigest()


def greedy_pick(logits):
    """The scan of greedy_sample (src/gten/sampler.cpp:30-38): max starts at
    -inf and index 0, and a value is taken only when `val > max`."""
    x = np.where(np.isnan(logits), -np.inf, logits)
    return int(np.argmax(x)) if np.any(x > -np.inf) else 0


def record(name, w, full_logits=False):
    ref = OL.Reference()
    cfg = config_of(w)
    t0 = time.time()
    m = ref.model_create(cfg, w["seed"])
    if w.get("emb_scale"):
        # the synthetic weights with the embedding's deltas scaled, read
        # by the reference's own .gten reader
        path = os.path.join(tempfile.mkdtemp(), "w.gten")
        G.write(path, cfg, w["seed"], OL.Oracle(), payload_fn=G.scaled_embedding(w["emb_scale"], cfg.wdtype == OL.Q8))
        assert ref.model_load_gten(m, os.fsencode(path)) == 0
        os.remove(path)
    prompt = prompt_of(w)
    adt = OL.F16 if w["wdtype"] == OL.F16 else OL.Q8
    rb = OL.row_bytes(adt, cfg.n_embd)

    def layer_digests(row):
        out = []
        for l in range(cfg.n_layers):
            p = ref.model_layer_out(m, l, row)
            out.append(sha(np.ctypeslib.as_array((OL.C.c_uint8 * rb).from_address(p))))
        return out

    logits = np.zeros(cfg.n_vocab, np.float32)
    ref.model_logits(m, OL.ptr(prompt), len(prompt), 0, OL.ptr(logits))
    prefill = logits.copy()
    layers = layer_digests(len(prompt) - 1)
    top = np.argsort(-prefill, kind="stable")[:16]
    # greedy_sample's loop, step by step
    toks = [int(t) for t in prompt]
    gen, steps = [], []
    for i in range(w["gen"]):
        if i > 0:
            seq = np.array(toks, np.int32)
            ref.model_logits(m, OL.ptr(seq), len(seq), len(seq) - 1, OL.ptr(logits))
        t = greedy_pick(logits)
        last = i == w["gen"] - 1 or t == cfg.eos
        if i > 0 and (i in DIGEST_STEPS or last):
            steps.append(dict(step=i, pos=len(toks) - 1, logits_sha256=sha(logits),
                              layer_out_sha256=layer_digests(len(toks) - 1)))
        if t == cfg.eos:
            break
        gen.append(t)
        toks.append(t)
    ref.model_free(m)
    fx = dict(workload=name, seed=w["seed"], prompt=prompt.tolist(), tokens=gen,
              prefill_logits_sha256=sha(prefill), layer_out_sha256=layers,
              prefill_top=[[int(i), float(prefill[i])] for i in top], decode_steps=steps,
              seconds=round(time.time() - t0, 1))
    with open(os.path.join(HERE, f"{name}.json"), "w") as f:
        json.dump(fx, f)
    if full_logits:
        np.save(os.path.join(HERE, f"{name}.prefill_logits.npy"), prefill)
    print(name, len(gen), "tokens", fx["seconds"], "s", flush=True)


# top-k / temperature runs: (temp, top_k, seed); temp 2.5 is clamped to 2.0
# and top_k 5000 to 1000 as the reference clamps them
TOPK_SMALL = [(0.8, 40, 7), (1.0, 1000, 11), (2.5, 5, 99), (0.6, 5000, 3)]
TOPK_FULL = [(0.8, 40, 7), (1.0, 1000, 11)]
TOPK_FULL_WORKLOADS = ["tinyllama-q4", "minicpm-q4"]


def record_topk(name, w, runs, n_gen):
    """topk_sample's loop with std::mt19937(seed), per run."""
    ref = OL.Reference()
    cfg = config_of(w)
    prompt = prompt_of(w)
    out = np.zeros(n_gen, np.int32)
    recs = []
    t0 = time.time()
    for temp, k, seed in runs:
        m = ref.model_create(cfg, w["seed"])
        n = ref.generate_topk(m, OL.ptr(prompt), len(prompt), n_gen, temp, k, seed, OL.ptr(out))
        ref.model_free(m)
        recs.append(dict(temp=temp, top_k=k, seed=seed, n_gen=n_gen, tokens=out[:n].tolist()))
    with open(os.path.join(HERE, f"{name}.topk.json"), "w") as f:
        json.dump(dict(workload=name, prompt=prompt.tolist(), runs=recs), f)
    print(name, "top-k", [len(r["tokens"]) for r in recs], round(time.time() - t0, 1), "s", flush=True)


def main(argv):
    if argv[:1] == ["--topk"]:
        for name in argv[1:] or list(SMALL) + TOPK_FULL_WORKLOADS:
            if name in SMALL:
                record_topk(name, SMALL[name], TOPK_SMALL, SMALL[name]["gen"])
            else:
                record_topk(name, nc.WORKLOADS[name], TOPK_FULL, 64)
        return
    models = dict(SMALL, **WIDE, **LONG)
    names = argv or list(models) + list(nc.WORKLOADS)
    for name in names:
        if name in models:
            record(name, models[name], full_logits=name in SMALL)
        else:
            record(name, nc.WORKLOADS[name], full_logits=name == "tinyllama-q4")


if __name__ == "__main__":
    main(sys.argv[1:])
