"""Tree reduction mode of the decode step (nc_model_set_reduce).

The tree mode replaces three sequential fp32 sums of the fused Q8/Q4 decode
kernels -- rms_norm's sum of squares, each matvec row's block/lane chains and
the softmax denominator -- with tree reductions.  Its results are no longer
the reference's bits; the ordered mode, which is bit-exact (the other GPU
tests), is the yardstick.

What is tested here, on models at the workloads' widths and two or three
layers deep: a tree step leaves every requantized code of the ordered step
in place, or (where one rounds the other way) stays within a loose bound.  What does not hold: once a reordered sum rounds one requantized
code the other way, every output of the next matvec moves by a few percent
of a code step and a share of them round the other way too, so the
difference spreads through the Q8 activations of every later layer.  In
TinyLlama's 22 layers (bench.py, step_vs_ordered) the logits end up ~4%
apart, so the tree mode does not meet a 1e-3 bound at the workloads' depth.
"""
import json
import os

import numpy as np
import pytest

import oracle_lib as OL
from nc_pkg import nc
from workloads import ALL, SMALL, config_of, prompt_of

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
# Models at the workloads' widths but two or three layers deep.  Their
# single-row steps run the fused decode kernels (the gate|up kernel is built
# for rows of 2048 and 2304 values), and at this depth the tree mode's
# reordered sums rarely move a requantized code.
WIDE = {
    "wide-llama-q4": dict(arch=nc.LLAMA, wdtype=nc.Q4, n_vocab=32000, n_embd=2048, n_layers=2, n_heads=32,
                          n_kv_heads=4, n_ffn=5632, eos=-1, rope_pct=1.0, prompt=16, gen=16, seed=0x7EE0001),
    "wide-llama-q8": dict(arch=nc.LLAMA, wdtype=nc.Q8, n_vocab=32000, n_embd=2048, n_layers=2, n_heads=32,
                          n_kv_heads=4, n_ffn=5632, eos=-1, rope_pct=1.0, prompt=16, gen=16, seed=0x7EE0002),
    # MiniCPM's own vocabulary: its tied lm head runs the row-chain kernel
    "wide-minicpm-q4": dict(arch=nc.MINICPM, wdtype=nc.Q4, n_vocab=122753, n_embd=2304, n_layers=2, n_heads=36,
                            n_kv_heads=36, n_ffn=5760, eos=-1, rope_pct=1.0, prompt=16, gen=16, seed=0x7EE0003),
    "wide-openelm-q8": dict(arch=nc.OPENELM, wdtype=nc.Q8, n_vocab=32000, n_embd=2048, n_layers=3,
                            n_heads=[16, 16, 20], n_kv_heads=[4, 4, 5], n_ffn=[1024, 4608, 8192], eos=-1,
                            rope_pct=1.0, prompt=16, gen=16, seed=0x7EE0004),
}


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def deq_q8_row(ref_bytes, cols):
    """A Q8 Act row in the reference's layout (per 32 values: fp16 delta,
    32 int8 codes) as fp32 values."""
    blk = np.frombuffer(np.ascontiguousarray(ref_bytes).tobytes(), np.uint8).reshape(-1, 34)[: (cols + 31) // 32]
    d = blk[:, :2].copy().view(np.float16).astype(np.float32)
    q = blk[:, 2:].copy().view(np.int8).astype(np.float32)
    return (q * d).reshape(-1)[:cols]


def golden(name):
    with open(os.path.join(GOLDEN, f"{name}.json")) as f:
        return json.load(f)


def codes_of(ref_bytes):
    return np.frombuffer(np.ascontiguousarray(ref_bytes).tobytes(), np.uint8).reshape(-1, 34)[:, 2:]


@pytest.mark.parametrize("name", list(WIDE))
def test_tree_step_against_ordered(gpu, oracle, name):
    """One decode step in both modes on the same cache; the ordered one
    equals the oracle's logits bit for bit.  Where the tree step's
    requantized codes all equal the ordered step's -- every code of every
    layer's rows, which a dropped, doubled or misplaced term in a tree fold
    or sum would not leave in place -- its logits differ from the ordered
    ones only by the lm head's own reordered fold (rel-L2 <= 1e-5).  Where a code
    moved, the change spreads through the later Q8 rows (wide-llama-q4: 921
    codes of layer 1's row, rel-L2 0.013); the test then only bounds it
    (rel-L2 <= 0.05)."""
    w = WIDE[name]
    cfg = config_of(w)
    prompt = prompt_of(w)
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig))
    m.init_synthetic(w["seed"])
    logits = m.logits(prompt, 0)
    seq = np.concatenate([prompt, [int(np.argmax(logits))]]).astype(np.int32)
    n = len(seq)
    ordered = m.logits(seq, n - 1)
    # the ordered step (fused kernels at full width, the lm head's
    # row-chain kernel) equals the oracle bit for bit
    om = oracle.model_create(cfg, w["seed"])
    o_logits = np.zeros(cfg.n_vocab, np.float32)
    oracle.model_logits(om, OL.ptr(prompt), len(prompt), 0, OL.ptr(o_logits))
    oracle.model_logits(om, OL.ptr(seq), n, n - 1, OL.ptr(o_logits))
    oracle.model_free(om)
    assert np.array_equal(ordered.view(np.uint32), o_logits.view(np.uint32)), \
        f"ordered step rel-L2 {rel_l2(ordered, o_logits):.3g}"
    rows_ord = [m.layer_out(l, n - 1) for l in range(cfg.n_layers)]
    m.set_reduce(gpu.REDUCE_TREE)
    tree = m.logits(seq, n - 1)
    rows_tree = [m.layer_out(l, n - 1) for l in range(cfg.n_layers)]
    errs = [rel_l2(deq_q8_row(t, cfg.n_embd), deq_q8_row(o, cfg.n_embd)) for t, o in zip(rows_tree, rows_ord)]
    moved = [int((codes_of(t) != codes_of(o)).sum()) for t, o in zip(rows_tree, rows_ord)]
    e = rel_l2(tree, ordered)
    print(f"{name}: logits rel-L2 {e:.3g}, layer rows {[f'{x:.3g}' for x in errs]}, codes moved {moved}", flush=True)
    if any(moved):
        assert max(errs) <= 0.05 and e <= 0.05
    else:
        # same codes in every layer: the logits differ only by the lm head's
        # own fold order (a tree in k_dmv; the row-chain kernel of tall Q4
        # heads folds in the reference's order in both modes)
        assert max(errs) == 0.0 and e <= 1e-5

    # back to the ordered mode: the ordered step's bits again
    m.set_reduce(gpu.REDUCE_ORDERED)
    again = m.logits(seq, n - 1)
    assert np.array_equal(again.view(np.uint32), ordered.view(np.uint32))
    m.close()


@pytest.mark.parametrize("name", ["small-llama-q4", "small-zephyr-q8"])
def test_tree_mode_leaves_unfused_paths_ordered(gpu, name):
    """Models whose steps do not run the fused kernels (rows other than
    2048 / 2304 values, layer_norm) keep the reference's stream bit for bit
    in the tree mode."""
    w = SMALL[name]
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig))
    m.init_synthetic(w["seed"])
    m.set_reduce(gpu.REDUCE_TREE)
    assert m.generate(prompt_of(w), w["gen"]).tolist() == golden(name)["tokens"]
    m.close()


