"""Model-level parity of the HIP decode path through the C-ABI.

Small models of every architecture: device weights, prefill logits, every
layer's residual row and the greedy stream must equal the oracle's and the
golden fixtures made by the reference (tests/golden/).  Every model with a
fixture -- small, full-width, long-context and the five full-size
workloads -- replays the reference's greedy loop step by step: the prefill
digests, and at the recorded decode steps the digests of the step's fp32
logits and of every layer's residual row, must equal the reference's, and
the greedy stream (also through the captured step graph) must equal its
stream.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle_lib as OL
from workloads import ALL, LONG, SMALL, WIDE, config_of, prompt_of

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


FULL = ["tinyllama-q4", "tinyllama-q8", "openelm-q8", "zephyr-f16", "minicpm-q4", "tinyllama-f16", "zephyr-q4",
        "openelm-sm-q8", "openelm-md-q8", "zephyr-q8", "minicpm-q8", "minicpm-f16"]


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


def greedy_pick(logits):
    """greedy_sample's scan (src/gten/sampler.cpp:30-38): max from -inf,
    index 0, a value taken only when `val > max`."""
    x = np.where(np.isnan(logits), -np.inf, logits)
    return int(np.argmax(x)) if np.any(x > -np.inf) else 0


@pytest.mark.parametrize("name", list(SMALL) + list(WIDE) + list(LONG) + FULL)
def test_decode_steps_match_reference(gpu, oracle, name):
    """The reference's greedy loop replayed through Model::logits (start_pos
    = n - 1 after the prompt), every step a fused (or op-by-op) decode step
    with direct launches: at the recorded steps the fp32 logits and every
    layer's row at the step's position equal the reference's bit for bit,
    and each step's greedy token is the reference's.  Then the same stream
    through the captured step graph."""
    reference_loop(gpu, name, oracle)


def workload_model(gpu, w, oracle=None):
    """The device model of a workload dict: synthetic weights, the embedding's
    deltas scaled when the workload has emb_scale."""
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig))
    m.init_synthetic(w["seed"])
    if w.get("emb_scale"):
        import gten_file as G
        m.set_weight(-1, OL.TID_EMB, G.workload_weight(oracle, config_of(w), w, -1, OL.TID_EMB))
    return m


def reference_loop(gpu, name, oracle=None):
    """Model::logits stepped as the reference's greedy loop (start_pos = n -
    1 after the prompt): the prefill digests, the recorded decode steps'
    logits and layer rows and every token must be the reference's; then the
    stream through the captured step graph."""
    w = ALL[name]
    g = golden(name)
    prompt = prompt_of(w)
    assert prompt.tolist() == g["prompt"]
    cfg = config_of(w)
    m = workload_model(gpu, w, oracle)
    logits = m.logits(prompt, 0)
    assert sha(logits) == g["prefill_logits_sha256"], "prefill logits"
    for l, digest in enumerate(g["layer_out_sha256"]):
        assert sha(m.layer_out(l, len(prompt) - 1)) == digest, f"prefill layer {l}"
    steps = {s["step"]: s for s in g["decode_steps"]}
    toks = prompt.tolist()
    ref = g["tokens"]
    seen = set()
    for i in range(w["gen"]):
        if i > 0:
            logits = m.logits(np.array(toks, np.int32), len(toks) - 1)
        if i in steps:
            s = steps[i]
            assert s["pos"] == len(toks) - 1
            assert sha(logits) == s["logits_sha256"], f"step {i} (position {s['pos']}): logits"
            for l, digest in enumerate(s["layer_out_sha256"]):
                assert sha(m.layer_out(l, len(toks) - 1)) == digest, f"step {i}: layer {l}"
            seen.add(i)
        t = greedy_pick(logits)
        if i == len(ref):
            assert t == cfg.eos
            break
        assert t == ref[i], f"step {i}: token {t}, reference {ref[i]}"
        toks.append(t)
    assert seen == set(steps)
    m.close()
    m = workload_model(gpu, w, oracle)
    assert m.generate(prompt, w["gen"]).tolist() == ref
    m.close()


@pytest.mark.parametrize("skew", [2.0, 1.001, 1.0 + 2.0 ** -22])
@pytest.mark.parametrize("name", ["wide-llama-q4", "wide-llama-q8", "wide-minicpm-q4", "wide-zephyr-q4", "wide-zephyr-q8",
                                  "tinyllama-q4"])
def test_speculative_norm_rows_recomputed(gpu, name, skew):
    """The fused norm launches compute their weight terms from a row
    normalized with a predicted sum of squares (rms_norm) or mean and
    variance (layer_norm), beside the exact sums, and recompute the blocks
    where the exact row differs.  A prediction skewed from the host makes
    rows differ (all blocks at 2x, some at 1.001x, the odd tie at
    1 + 2^-22): the fix-ups must run and every digest and token must still
    be the reference's."""
    L = gpu.lib()
    cnt = gpu.DeviceBuffer(4)
    cnt.upload(np.zeros(1, np.int32))
    gpu.check(L.nc_debug_spec(skew, cnt.ptr))
    try:
        reference_loop(gpu, name)
    finally:
        gpu.check(L.nc_debug_spec(1.0, None))
    fixups = int(cnt.download(np.zeros(1, np.int32))[0])
    cnt.close()
    if skew > 1.0005:
        assert fixups > 0, "the recomputation path did not run"


@pytest.mark.parametrize("max_ctx", [200, 1024, 4096])
@pytest.mark.parametrize("name", ["small-llama-q8", "small-zephyr-q8", "small-zephyr-q4"])
def test_small_model_stream_with_larger_cache(gpu, name, max_ctx):
    """Caches larger than the sequence (the attention kernels size their
    shared memory and prefetch by the cache) give the same varying streams,
    up to the reference's default context (1024) and the longest (4096)."""
    w = SMALL[name]
    g = golden(name)
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig, max_ctx=max_ctx))
    m.init_synthetic(w["seed"])
    assert m.generate(prompt_of(w), w["gen"]).tolist() == g["tokens"]
    m.close()


def test_full_workload_at_default_context(gpu):
    """TinyLlama-Q4 built with the reference's default inference context of
    1024 positions (src/nanochat.cpp:40, sampler.cpp:13): the fused decode
    step sized for it gives the workload's stream."""
    w = ALL["tinyllama-q4"]
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig, max_ctx=1024))
    m.init_synthetic(w["seed"])
    assert m.generate(prompt_of(w), w["gen"]).tolist() == golden("tinyllama-q4")["tokens"]
    m.close()


def test_context_limit(gpu):
    """max_ctx beyond the longest context of the reference's models is
    refused at creation, not at the first decode step."""
    w = SMALL["small-llama-q4"]
    with pytest.raises(gpu.HipError, match="max_ctx"):
        gpu.Model(config_of(w, cls=gpu.ModelConfig, max_ctx=gpu.MAX_CTX + 1))


def crafted_head(oracle, cfg, seed, layer, slot):
    """The synthetic lm head (or tied embedding) rewritten so that its logits
    hold NaN, +0 and exact ties for any input: rows 0-3 and 100-199 all-zero
    codes (logit +0), rows 4 and 17 NaN deltas (NaN logits), every other row
    a copy of row 6 (one shared logit, tied at every index)."""
    import gten_file as G
    rows, cols, dt = oracle.weight_shape(cfg, layer, slot)
    rb = OL.row_bytes(dt, cols)
    W = G.weight_bytes(oracle, cfg, seed, layer, slot).reshape(rows, rb).copy()
    W[:] = W[6]
    bsz = 18 if dt == OL.Q4 else 34
    blk = W.reshape(rows, cols // 32, bsz)
    zero = 0x77 if dt == OL.Q4 else 0x00  # Q4 code 7 is the value 0
    for r in list(range(0, 4)) + list(range(100, 200)):
        blk[r, :, 2:] = zero
    for r in (4, 17):
        blk[r, :, 0] = 0x00
        blk[r, :, 1] = 0x7E  # fp16 NaN delta
    return np.ascontiguousarray(W.reshape(-1))


@pytest.mark.parametrize("name", ["wide-llama-q4", "wide-llama-q8", "small-llama-q4", "wide-minicpm-q4"])
def test_greedy_pick_with_nan_and_tied_logits(gpu, oracle, name):
    """The greedy token of each decode step (the fused lm head's argmax
    epilogue for the wide models, k_argmax_advance after the op-by-op step of
    the small one) is greedy_sample's scan (src/gten/sampler.cpp:30-41) over
    logits holding NaN, +0 and exact ties: the first index of the largest
    non-NaN value.  The oracle runs the same model and scan."""
    w = ALL[name]
    cfg = config_of(w)
    slot = OL.TID_EMB if cfg.arch == OL.MINICPM else OL.TID_LM
    W = crafted_head(oracle, cfg, w["seed"], -1, slot)
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig))
    m.init_synthetic(w["seed"])
    m.set_weight(-1, slot, W)
    om = oracle.model_create(cfg, w["seed"])
    p = oracle.model_weight(om, -1, slot)
    OL.C.memmove(p, W.ctypes.data, W.nbytes)
    prompt = prompt_of(w)
    n_gen = 12
    logits = m.logits(prompt, 0)
    assert np.isnan(logits[4]) and np.isnan(logits[17]) and logits[100] == 0.0
    assert logits[5] == logits[8] == logits[6]
    want = np.zeros(n_gen, np.int32)
    n = oracle.generate_greedy(om, OL.ptr(prompt), len(prompt), n_gen, OL.ptr(want))
    oracle.model_free(om)
    got = m.generate(prompt, n_gen)
    m.close()
    assert got.tolist() == want[:n].tolist()
    # the first +0 row, or the first shared row (after the NaN row 4)
    assert set(got.tolist()) <= {0, 5}


@pytest.mark.parametrize("case", ["signed_zeros", "nan_first", "nan_between", "all_nan", "neg_inf"])
def test_argmax_nan_and_signed_zero(gpu, oracle, case):
    """nc_argmax (the prefill's greedy pick) over NaN, -inf and +-0: the
    first index of the largest value greedy_sample's `val > max` scan takes."""
    import ctypes as C
    from devutil import dev_array
    n = 5000
    rng = np.random.default_rng(3)
    x = -np.abs(rng.standard_normal(n)).astype(np.float32) - 1.0
    if case == "signed_zeros":
        x[10], x[20], x[30] = -0.0, 0.0, -0.0  # -0 ties with +0: index 10
    elif case == "nan_first":
        x[0], x[1], x[2] = np.nan, np.nan, -0.5
    elif case == "nan_between":
        x[100], x[101], x[4000] = 2.0, np.nan, 2.0
    elif case == "all_nan":
        x[:] = np.nan
    elif case == "neg_inf":
        x[:] = -np.inf
        x[4321] = np.nan
    dx = dev_array(x)
    out = np.zeros(1, np.int32)
    dout = dev_array(out)
    gpu.check(gpu.lib().nc_argmax(C.c_void_p(dx.ptr), n, C.c_void_p(dout.ptr), None), "argmax")
    dout.download(out)
    assert out[0] == oracle.argmax(OL.ptr(x), n) == greedy_pick(x)
