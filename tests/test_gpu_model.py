"""Model-level parity of the HIP decode path through the C-ABI.

Small models of every architecture: device weights, prefill logits, every
layer's residual row and the greedy stream must equal the oracle's and the
golden fixtures made by the reference (tests/golden/).  Full-size workloads:
the greedy stream and the prefill digests must equal the reference's golden
fixtures.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle_lib as OL
from workloads import ALL, SMALL, config_of, prompt_of

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name):
    path = os.path.join(GOLDEN, f"{name}.json")
    if not os.path.exists(path):
        pytest.fail(f"missing golden fixture {path}")
    with open(path) as f:
        return json.load(f)


def sha(b):
    return hashlib.sha256(np.ascontiguousarray(b).tobytes()).hexdigest()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def weight_slots(cfg):
    slots = [(-1, OL.TID_EMB), (-1, OL.TID_NORM), (-1, OL.TID_NORM_B), (-1, OL.TID_LM)]
    for l in range(cfg.n_layers):
        slots += [(l, s) for s in range(len(OL.W_SLOTS))]
    return slots


@pytest.mark.parametrize("name", list(SMALL))
def test_small_model_weights_bit_exact(gpu, oracle, name):
    w = SMALL[name]
    cfg = config_of(w)
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig))
    m.init_synthetic(w["seed"])
    for layer, slot in weight_slots(cfg):
        shape = oracle.weight_shape(cfg, layer, slot)
        if shape is None:
            continue
        rows, cols, dt = shape
        nbytes = rows * OL.row_bytes(dt, cols)
        want = np.zeros(nbytes, np.uint8)
        oracle.make_weight(OL.C.byref(cfg), w["seed"], layer, slot, OL.ptr(want))
        got = m.get_weight(layer, slot, nbytes)
        assert np.array_equal(got, want), (name, layer, slot)
    m.close()


@pytest.mark.parametrize("name", list(SMALL))
def test_small_model_prefill_and_stream(gpu, oracle, name):
    w = SMALL[name]
    g = golden(name)
    prompt = prompt_of(w)
    assert prompt.tolist() == g["prompt"]
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig))
    m.init_synthetic(w["seed"])
    logits = m.logits(prompt, 0)
    want = np.load(os.path.join(GOLDEN, f"{name}.prefill_logits.npy"))
    assert rel_l2(logits, want) <= 1e-3
    assert np.array_equal(logits.view(np.uint32), want.view(np.uint32)), f"rel-L2 {rel_l2(logits, want):.3g}"
    for l, digest in enumerate(g["layer_out_sha256"]):
        assert sha(m.layer_out(l, len(prompt) - 1)) == digest, f"layer {l}"
    # one decode step through the oracle on the same sequence
    cfg = config_of(w)
    om = oracle.model_create(cfg, w["seed"])
    seq = np.concatenate([prompt, [int(np.argmax(logits))]]).astype(np.int32)
    o_logits = np.zeros(cfg.n_vocab, np.float32)
    oracle.model_logits(om, OL.ptr(prompt), len(prompt), 0, OL.ptr(o_logits))
    oracle.model_logits(om, OL.ptr(seq), len(seq), len(seq) - 1, OL.ptr(o_logits))
    d_logits = m.logits(seq, len(seq) - 1)
    assert np.array_equal(d_logits.view(np.uint32), o_logits.view(np.uint32)), f"step rel-L2 {rel_l2(d_logits, o_logits):.3g}"
    oracle.model_free(om)
    toks = m.generate(prompt, w["gen"])
    assert toks.tolist() == g["tokens"]
    m.close()


FULL = ["tinyllama-q4", "tinyllama-q8", "openelm-q8", "zephyr-f16", "minicpm-q4"]


@pytest.mark.parametrize("name", FULL)
def test_full_workload_stream(gpu, name):
    """Greedy stream of the full-size workload equals the reference's."""
    w = ALL[name]
    g = golden(name)
    prompt = prompt_of(w)
    assert prompt.tolist() == g["prompt"]
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig))
    m.init_synthetic(w["seed"])
    logits = m.logits(prompt, 0)
    top = [[int(i), float(logits[i])] for i in np.argsort(-logits, kind="stable")[:16]]
    assert [t[0] for t in top] == [t[0] for t in g["prefill_top"]]
    layer_ok = [sha(m.layer_out(l, len(prompt) - 1)) == d for l, d in enumerate(g["layer_out_sha256"])]
    assert all(layer_ok), f"first differing layer {layer_ok.index(False)}"
    assert sha(logits) == g["prefill_logits_sha256"]
    toks = m.generate(prompt, w["gen"])
    ref = g["tokens"]
    first_diff = next((i for i, (a, b) in enumerate(zip(toks.tolist(), ref)) if a != b), None)
    assert toks.tolist() == ref, f"streams diverge at step {first_diff}"
    m.close()


@pytest.mark.parametrize("max_ctx", [200, 400])
@pytest.mark.parametrize("name", ["small-llama-q4", "small-openelm-q8"])
def test_small_model_stream_with_larger_cache(gpu, name, max_ctx):
    """The decode attention sizes its register prefetch to the cache: the
    cache sizes of no full workload (200, 400 positions) give the same
    stream."""
    w = SMALL[name]
    g = golden(name)
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig, max_ctx=max_ctx))
    m.init_synthetic(w["seed"])
    assert m.generate(prompt_of(w), w["gen"]).tolist() == g["tokens"]
    m.close()
