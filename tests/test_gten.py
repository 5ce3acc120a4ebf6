"""The .gten checkpoint path: Model::load_from_ckpt (tinyllama/tinyllama.cpp:
131-187, zephyr/zephyr.cpp:79-150, minicpm/minicpm.cpp:113-166,
openelm/openelm.cpp:201-262) reading records with gten::read_layer_header /
read_into_weight (gten/utils.cpp:29-61).

Files are written from the oracle's synthetic weights (tests/gten_file.py).
On the CPU the reference's own reader loads them into a model made with other
weights, and its greedy stream must equal the golden fixture of the seeded
model: the writer's record order is the reference's.  On the GPU the
product's loader must give device weights bit-equal to the oracle's and the
same golden stream, and must reject a wrong magic number, a payload size
that does not match the tensor, a truncated file and a missing one.
"""
import json
import os

import numpy as np
import pytest

import gten_file as G
import oracle_lib as OL
from workloads import SMALL, config_of, prompt_of

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden_tokens(name):
    with open(os.path.join(GOLDEN, f"{name}.json")) as f:
        return json.load(f)["tokens"]


def run_model(lib, m, cfg, w):
    """Prefill logits of the workload's prompt and its greedy stream."""
    prompt = prompt_of(w)
    logits = np.zeros(cfg.n_vocab, np.float32)
    lib.model_logits(m, OL.ptr(prompt), len(prompt), 0, OL.ptr(logits))
    out = np.zeros(w["gen"], np.int32)
    n = lib.generate_greedy(m, OL.ptr(prompt), len(prompt), w["gen"], OL.ptr(out))
    return logits, out[:n].tolist()


def oracle_with(oracle, cfg, seed, pl):
    """The oracle's model with every weight replaced, by (layer, slot), from
    the payload dict pl."""
    m = oracle.model_create(cfg, seed)
    for (layer, slot), data in pl.items():
        p = oracle.model_weight(m, layer, slot)
        assert p, (layer, slot)
        OL.C.memmove(p, data, len(data))
    return m


@pytest.mark.parametrize("name", list(SMALL))
def test_written_file_layout(oracle, tmp_path, name):
    """Record count, names and payload sizes follow the model's file order;
    payloads are the reference storage of each weight."""
    w = SMALL[name]
    cfg = config_of(w)
    path = str(tmp_path / "m.gten")
    G.write(path, cfg, w["seed"], oracle)
    magic, recs = G.read(path)
    assert magic == G.MAGIC
    assert magic.to_bytes(8, "little") == b"GTENFILE"
    order = G.order(cfg)
    per_layer = {OL.LLAMA: 9, OL.ZEPHYR: 14, OL.MINICPM: 9, OL.OPENELM: 11}[cfg.arch]
    tail = {OL.LLAMA: 2, OL.ZEPHYR: 3, OL.MINICPM: 1, OL.OPENELM: 1}[cfg.arch]
    assert len(recs) == len(order) == 1 + per_layer * cfg.n_layers + tail
    for (layer, slot, name_), (lname, wname, data) in zip(order, recs):
        assert lname == wname == name_
        rows, cols, dt = oracle.weight_shape(cfg, layer, slot)
        assert len(data) == rows * OL.row_bytes(dt, cols)
        assert data == G.weight_bytes(oracle, cfg, w["seed"], layer, slot).tobytes()


@pytest.mark.parametrize("name", list(SMALL))
def test_reference_reader_loads_written_file(oracle, reference, tmp_path, name):
    """The reference's read_layer_header / read_into_weight, in each model's
    load_from_ckpt order, turn a model made from another seed into the
    seeded one: its greedy stream equals the golden fixture."""
    w = SMALL[name]
    cfg = config_of(w)
    path = str(tmp_path / "m.gten")
    G.write(path, cfg, w["seed"], oracle)
    m = reference.model_create(cfg, w["seed"] + 1000)
    assert reference.model_load_gten(m, os.fsencode(path)) == 0
    prompt = prompt_of(w)
    out = np.zeros(w["gen"], np.int32)
    n = reference.generate_greedy(m, OL.ptr(prompt), len(prompt), w["gen"], OL.ptr(out))
    reference.model_free(m)
    assert out[:n].tolist() == golden_tokens(name)


@pytest.mark.parametrize("name", list(SMALL))
def test_reference_reader_order_with_distinct_norms(oracle, reference, tmp_path, name):
    """Every norm gain and bias distinct: the model the reference reads from
    the file computes bit-equal logits and the same stream as the oracle
    with the same tensors placed by (layer, slot)."""
    w = SMALL[name]
    cfg = config_of(w)
    pl = G.payloads(cfg, w["seed"], oracle, G.distinct_vectors)
    path = str(tmp_path / "m.gten")
    G.write(path, cfg, w["seed"], oracle, payload_fn=G.distinct_vectors)
    rm = reference.model_create(cfg, w["seed"] + 1000)
    assert reference.model_load_gten(rm, os.fsencode(path)) == 0
    r_logits, r_toks = run_model(reference, rm, cfg, w)
    reference.model_free(rm)
    om = oracle_with(oracle, cfg, w["seed"], pl)
    o_logits, o_toks = run_model(oracle, om, cfg, w)
    oracle.model_free(om)
    assert np.array_equal(r_logits.view(np.uint32), o_logits.view(np.uint32))
    assert r_toks == o_toks
    # the distinct norms change the model: its logits are not the seeded model's
    plain = np.load(os.path.join(GOLDEN, f"{name}.prefill_logits.npy"))
    assert not np.array_equal(r_logits.view(np.uint32), plain.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(SMALL))
def test_load_gten_weights_and_stream(gpu, oracle, tmp_path, name):
    """The synthetic model's file: the golden stream.  A file with distinct
    norm gains and biases: device weights equal to the file's tensors, and
    prefill logits and stream equal to the oracle's with those tensors."""
    w = SMALL[name]
    cfg = config_of(w)
    path = str(tmp_path / "m.gten")
    G.write(path, cfg, w["seed"], oracle)
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig))
    m.init_synthetic(w["seed"] + 1000)
    m.load_gten(path)
    assert m.generate(prompt_of(w), w["gen"]).tolist() == golden_tokens(name)

    pl = G.payloads(cfg, w["seed"], oracle, G.distinct_vectors)
    G.write(path, cfg, w["seed"], oracle, payload_fn=G.distinct_vectors)
    m.load_gten(path)
    for (layer, slot), data in pl.items():
        got = m.get_weight(layer, slot, len(data))
        assert got.tobytes() == data, (name, layer, slot)
    om = oracle_with(oracle, cfg, w["seed"], pl)
    o_logits, o_toks = run_model(oracle, om, cfg, w)
    oracle.model_free(om)
    logits = m.logits(prompt_of(w), 0)
    assert np.array_equal(logits.view(np.uint32), o_logits.view(np.uint32))
    assert m.generate(prompt_of(w), w["gen"]).tolist() == o_toks
    m.close()


@pytest.mark.gpu
def test_load_gten_rejects_bad_files(gpu, oracle, tmp_path):
    w = SMALL["small-llama-q4"]
    cfg = config_of(w)
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig))

    def expect_error(path, text):
        with pytest.raises(gpu.HipError, match=text):
            m.load_gten(path)

    expect_error(str(tmp_path / "absent.gten"), "cannot open")
    p = str(tmp_path / "magic.gten")
    G.write(p, cfg, w["seed"], oracle, magic=G.MAGIC ^ 1)
    expect_error(p, "Magic number")
    # one payload two bytes short: the reference's size assertion
    p = str(tmp_path / "size.gten")
    G.write(p, cfg, w["seed"], oracle,
            payload_fn=lambda layer, slot, d: d[:-2] if (layer, slot) == (1, G.W_UP) else d)
    expect_error(p, r"Weight `model\.layers\.1\.mlp\.up_proj\.weight` data size")
    # files cut inside a header and inside a payload
    full = str(tmp_path / "full.gten")
    G.write(full, cfg, w["seed"], oracle)
    size = os.path.getsize(full)
    first = 8 + 2 * (4 + len("model.embed_tokens.weight"))  # offset of the first payload size
    for cut, text in ((4, "Magic number"), (8 + 2, "ends before tensor"), (first + 2, "ends before tensor"),
                      (size - 5, "ends inside weight `lm_head.weight`")):
        p = str(tmp_path / f"cut{cut}.gten")
        G.write(p, cfg, w["seed"], oracle, truncate=cut)
        expect_error(p, text)
    # the complete file still loads into the same model afterwards
    m.load_gten(full)
    assert m.generate(prompt_of(w), w["gen"]).tolist() == golden_tokens("small-llama-q4")
    m.close()
