"""Pins the oracle (CPU restatement) before it is trusted as the checker.

* against the reference's own code (oracle/_ref, compiled from its sources)
  on random inputs of every op, and on whole small models;
* against the golden fixtures the reference wrote (tests/golden/);
* against closed forms and independent libraries where the mathematics fixes
  the answer (numpy's IEEE fp16 conversions, hand-derived rounding cases that
  a wrong lane order or rounding rule would fail).
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle_lib as OL
from workloads import SMALL, config_of, prompt_of

Q8, Q4, F16, F32 = OL.Q8, OL.Q4, OL.F16, OL.F32
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def q8_rows(oracle, x):
    rows, cols = x.shape
    out = np.zeros((rows, OL.row_bytes(Q8, cols)), np.uint8)
    for r in range(rows):
        oracle.q8_quantize_row(OL.ptr(np.ascontiguousarray(x[r])), OL.ptr(out[r]), cols)
    return out


def block(delta16, codes):
    """One reference Q8 block: fp16 delta bits + 32 int8 codes."""
    b = np.zeros(34, np.uint8)
    b[:2] = np.array([delta16], np.uint16).view(np.uint8)
    b[2:] = np.array(codes, np.int8).view(np.uint8)
    return b


# ------------------------------------------------------------ conversions --

def test_fp16_to_fp32_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([oracle.fp16_to_fp32(int(v)) for v in h], np.float32)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_fp32_to_fp16_rne(oracle):
    rng = np.random.default_rng(0)
    halves = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    nxt = np.nextafter(halves, np.float32(np.inf))
    mids = ((halves.astype(np.float64) + np.roll(halves, -1).astype(np.float64)) / 2)[:-1].astype(np.float32)
    cases = np.concatenate([halves, -halves, mids, -mids, nxt, rng.standard_normal(20000).astype(np.float32) * 100,
                            np.float32([65504, 65519.99, 65520, 65536, 1e-8, 2.98e-8, 5.96e-8, 6.1e-5])])
    got = np.array([oracle.fp32_to_fp16(float(v)) for v in cases], np.uint16)
    want = cases.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_fp16_conversions_match_reference(oracle, reference):
    rng = np.random.default_rng(1)
    for h in range(0, 65536, 7):
        a, b = oracle.fp16_to_fp32(h), reference.fp16_to_fp32(h)
        assert (np.isnan(a) and np.isnan(b)) or np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)
    for f in np.concatenate([rng.standard_normal(5000) * 1000, rng.standard_normal(5000) * 1e-5]).astype(np.float32):
        assert oracle.fp32_to_fp16(float(f)) == reference.fp32_to_fp16(float(f))


# -------------------------------------------------------------- quantizers --

def test_activation_quantizer_rounds_half_away(oracle):
    # absmax 127 -> delta 1.0 (fp16 0x3C00), scale 1.0: x * scale = x exactly
    x = np.zeros(32, np.float32)
    x[:8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.49, 3.5]
    out = np.zeros(34, np.uint8)
    oracle.q8_quantize_row(OL.ptr(x), OL.ptr(out), 32)
    assert out[:2].view(np.uint16)[0] == 0x3C00
    assert out[2:10].view(np.int8).tolist() == [127, 3, -3, 1, -1, 2, -1, 4]


def test_activation_quantizer_partial_block_and_zero(oracle):
    x = np.array([0.0] * 32 + [1.0, -2.0, 0.25], np.float32)
    out = np.zeros(2 * 34, np.uint8)
    oracle.q8_quantize_row(OL.ptr(x), OL.ptr(out), len(x))
    assert out[:2].view(np.uint16)[0] == 0 and not out[2:34].any()  # zero block: delta 0, scale 0
    d = np.float32(2.0) / np.float32(127.0)
    assert out[34:36].view(np.uint16)[0] == np.float16(d).view(np.uint16)
    s = np.float32(1.0) / d
    want = [int(np.trunc(v * s + np.copysign(0.5, v))) for v in (np.float32(1.0), np.float32(-2.0), np.float32(0.25))]
    assert out[36:39].view(np.int8).tolist() == want


def test_activation_quantizer_matches_reference(oracle, reference):
    rng = np.random.default_rng(2)
    for n in [1, 7, 31, 32, 33, 64, 95, 2048, 5632]:
        x = (rng.standard_normal(n) * rng.choice([1e-3, 1.0, 300.0])).astype(np.float32)
        x[::5] = np.round(x[::5] * 4) / 4  # many exact ties after scaling
        a = np.zeros(OL.row_bytes(Q8, n), np.uint8)
        b = np.zeros_like(a)
        oracle.q8_quantize_row(OL.ptr(x), OL.ptr(a), n)
        reference.q8_quantize_row(OL.ptr(x), OL.ptr(b), n)
        assert np.array_equal(a, b), n


def test_weight_quantizers_round_half_even_and_pack(oracle):
    x = np.zeros(32, np.float32)
    x[:6] = [127.0, 2.5, -2.5, 3.5, 0.5, -0.5]
    q8 = np.zeros(34, np.uint8)
    oracle.q8_quantize_weights(OL.ptr(x), 1, OL.ptr(q8))
    assert q8[:2].view(np.uint16)[0] == 0x3C00
    assert q8[2:8].view(np.int8).tolist() == [127, 2, -2, 4, 0, 0]  # torch.round: half to even
    # Q4: absmax 7 -> delta 1; codes = round(x) + 7; byte j = code(j) << 4 | code(j + 16)
    y = np.zeros(32, np.float32)
    y[0], y[1], y[16], y[17], y[31] = 7.0, 2.5, -7.0, 1.5, -0.5
    q4 = np.zeros(18, np.uint8)
    oracle.q4_quantize_weights(OL.ptr(y), 1, OL.ptr(q4))
    assert q4[:2].view(np.uint16)[0] == 0x3C00
    codes = q4[2:]
    assert codes[0] == (14 << 4) | 0 and codes[1] == (9 << 4) | 9 and codes[15] == (7 << 4) | 7
    assert all(c == 0x77 for c in codes[2:15])


def test_weight_quantizer_error_bound(oracle):
    """Stored delta = fp16(absmax / qmax) and every code reconstructs its value
    to within half a step (plus the fp16 rounding of the delta)."""
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    for dt, qmax in [(Q8, 127), (Q4, 7)]:
        out = np.zeros((64, OL.row_bytes(dt, 256)), np.uint8)
        (oracle.q8_quantize_weights if dt == Q8 else oracle.q4_quantize_weights)(OL.ptr(w), 64 * 8, OL.ptr(out))
        blocks = w.reshape(-1, 32)
        delta = (np.abs(blocks).max(1) / np.float32(qmax)).astype(np.float32)
        raw = out.reshape(-1, 34 if dt == Q8 else 18)
        d16 = raw[:, :2].copy().view(np.uint16).reshape(-1)
        assert np.array_equal(d16, delta.astype(np.float16).view(np.uint16))
        deq = np.zeros((64, 256), np.float32)
        for r in range(64):
            oracle.read_row(OL.ptr(out[r]), dt, OL.ptr(deq[r]), 256)
        err = np.abs(deq.reshape(-1, 32) - blocks)
        dq = d16.view(np.float16).astype(np.float32)
        bound = 0.5 * delta + qmax * np.abs(dq - delta) + 1e-9
        assert (err <= bound[:, None]).all()


# ----------------------------------------------------- dot-product structure --

def test_q8_dot_lane_structure_closed_form(oracle):
    """Lane k sums elements with (j mod 8) in {2k, 2k+1}; lanes fold in block
    order and finish as (l0 + l1) + (l2 + l3).  Deltas are powers of two so
    every term is exact and only the summation order rounds."""
    one = 0x3C00
    big = 0x6C00  # 4096.0: with code 127 * 127 * 4096 * 1 ~ 2^26
    a0 = [0] * 32
    a0[0] = 127  # lane 0, block 0: +127*127*4096
    a0[2] = -127  # lane 1, block 0: -127*127*4096
    a1 = [0] * 32
    a1[1] = 1  # lane 0, block 1: +1 (lost: acc0 = 66064384 + 1 rounds back)
    b0 = [0] * 32
    b0[0], b0[2] = 127, 127
    b1 = [0] * 32
    b1[1] = 1
    A = np.concatenate([block(big, a0), block(one, a1)])
    B = np.concatenate([block(one, b0), block(one, b1)])
    got = oracle.dot(OL.ptr(A), Q8, OL.ptr(B), Q8, 64)
    # exact sum is 1; the reference's order gives (66064384 + 1 -> 66064384) + (-66064384) = 0
    assert got == 0.0
    # same magnitudes in lanes 2/3 instead of 0/1 give the same structure
    a0b = [0] * 32
    a0b[4], a0b[6] = 127, -127
    b0b = [0] * 32
    b0b[4], b0b[6] = 127, 127
    a1b = [0] * 32
    a1b[12] = 1  # element 12: lane 2 again (12 mod 8 = 4)
    b1b = [0] * 32
    b1b[12] = 1
    A = np.concatenate([block(big, a0b), block(one, a1b)])
    B = np.concatenate([block(one, b0b), block(one, b1b)])
    assert oracle.dot(OL.ptr(A), Q8, OL.ptr(B), Q8, 64) == 0.0
    # put the +1 in lane 1 instead: (66064384 + (-66064384 + 1)) = 1 exactly representable? no:
    # -66064384 + 1 = -66064383 is not representable (ulp 4) -> -66064384, sum 0; use lane 2:
    a1c = [0] * 32
    a1c[5] = 1  # element 5: lane 2
    b1c = [0] * 32
    b1c[5] = 1
    A = np.concatenate([block(big, a0), block(one, a1c)])
    B = np.concatenate([block(one, b0), block(one, b1c)])
    assert oracle.dot(OL.ptr(A), Q8, OL.ptr(B), Q8, 64) == 1.0  # (x + -x) + (1 + 0)


def test_f32_dot_lanes_then_tail(oracle):
    # lanes: index mod 8; lane sum left to right; tail added after
    a = np.zeros(9, np.float32)
    b = np.ones(9, np.float32)
    a[0], a[1], a[8] = 1.0, 2 ** 24, 1.0
    # lanes: f0 + f1 = 1 + 2^24 rounds to 2^24; the tail 1 is added after the
    # lane sum and rounds away again (folding it into lane 0 would give 2^24 + 2)
    assert oracle.dot(OL.ptr(a), F32, OL.ptr(b), F32, 9) == 2.0 ** 24
    a[0], a[1], a[8] = 1.0, 1.0, 2 ** 24
    assert oracle.dot(OL.ptr(a), F32, OL.ptr(b), F32, 9) == 2.0 ** 24 + 2


# --------------------------------------------- ops against the reference code --

def _rand_act(oracle, rng, dt, rows, cols, scale=1.0):
    x = (rng.standard_normal((rows, cols)) * scale).astype(np.float32)
    if dt == F16:
        return x.astype(np.float16).view(np.uint16)
    return q8_rows(oracle, x)


def _rand_w(oracle, rng, dt, rows, cols):
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    if dt == F16:
        return w.astype(np.float16).view(np.uint16)
    out = np.zeros((rows, OL.row_bytes(dt, cols)), np.uint8)
    (oracle.q8_quantize_weights if dt == Q8 else oracle.q4_quantize_weights)(OL.ptr(w), rows * cols // 32, OL.ptr(out))
    return out


@pytest.mark.parametrize("xdt,wdt,odt", [(Q8, Q4, Q8), (Q8, Q8, Q8), (F16, F16, F16), (Q8, Q4, F32), (F16, F16, F32)])
@pytest.mark.parametrize("P,K,N,sp", [(1, 64, 64, 0), (5, 256, 96, 0), (6, 2048, 160, 5), (2, 5632, 64, 1)])
def test_matmul_matches_reference(oracle, reference, xdt, wdt, odt, P, K, N, sp):
    rng = np.random.default_rng(P * K + N)
    x = _rand_act(oracle, rng, xdt, P, K)
    w = _rand_w(oracle, rng, wdt, N, K)
    a = np.zeros((P, OL.row_bytes(odt, N)), np.uint8)
    b = np.zeros_like(a)
    oracle.matmul(OL.ptr(x), xdt, OL.ptr(w), wdt, OL.ptr(a), odt, K, N, sp, P, None)
    reference.matmul(OL.ptr(x), xdt, OL.ptr(w), wdt, OL.ptr(b), odt, K, N, sp, P)
    assert np.array_equal(a[sp:], b[sp:])


@pytest.mark.parametrize("dt", [Q8, F16])
@pytest.mark.parametrize("op", ["rms", "rms_heads", "ln", "silu", "scale", "bias", "rope", "rope25", "add", "mul"])
def test_elementwise_ops_match_reference(oracle, reference, dt, op):
    rng = np.random.default_rng(["rms", "rms_heads", "ln", "silu", "scale", "bias", "rope", "rope25", "add",
                                 "mul"].index(op) + 10 * dt)
    P, d = 7, 2048
    x = _rand_act(oracle, rng, dt, P, d, 3.0)
    y = _rand_act(oracle, rng, dt, P, d, 1.0)
    w = (1 + 0.1 * rng.standard_normal(d)).astype(np.float16).view(np.uint16)
    bb = (0.1 * rng.standard_normal(d)).astype(np.float16).view(np.uint16)
    o1, o2 = np.zeros_like(x), np.zeros_like(x)
    for lib, o in ((oracle, o1), (reference, o2)):
        if op == "rms":
            lib.rms_norm(OL.ptr(x), dt, OL.ptr(w), OL.ptr(o), d, 2, P)
        elif op == "rms_heads":
            lib.rms_norm_heads(OL.ptr(x), dt, OL.ptr(w), OL.ptr(o), d // 64, 64, 1, P)
        elif op == "ln":
            lib.layer_norm(OL.ptr(x), dt, OL.ptr(w), OL.ptr(bb), OL.ptr(o), d, 2, P)
        elif op == "silu":
            lib.silu(OL.ptr(x), OL.ptr(o), dt, d, 1, P)
        elif op == "scale":
            o[:] = x
            lib.scale(OL.ptr(o), dt, 0.2213594, d, 0, P)
        elif op == "bias":
            o[:] = x
            lib.bias_add(OL.ptr(o), dt, OL.ptr(bb), d, 0, P)
        elif op in ("rope", "rope25"):
            lib.rotary_emb(OL.ptr(x.copy()), OL.ptr(o), dt, d, 64, 1.0 if op == "rope" else 0.25, 3, P)
        elif op == "add":
            lib.add(OL.ptr(x), OL.ptr(y), OL.ptr(o), dt, d, 0, P)
        else:
            lib.multiply(OL.ptr(x), OL.ptr(y), OL.ptr(o), dt, d, 0, P)
    start = {"rms": 2, "ln": 2, "silu": 1, "rope": 3, "rope25": 3, "rms_heads": 1}.get(op, 0)
    assert np.array_equal(o1[start:], o2[start:])


@pytest.mark.parametrize("dt", [Q8, F16])
@pytest.mark.parametrize("n,sp,hq,hkv", [(1, 0, 4, 1), (9, 8, 4, 2), (37, 0, 8, 2), (70, 69, 32, 4), (33, 0, 2, 2),
                                         (200, 199, 8, 8)])
def test_attention_matches_reference(oracle, reference, dt, n, sp, hq, hkv):
    rng = np.random.default_rng(n * 100 + hq)
    q = _rand_act(oracle, rng, dt, n, hq * 64, 2.0)
    k = _rand_act(oracle, rng, dt, n, hkv * 64, 2.0)
    v = _rand_act(oracle, rng, dt, n, hkv * 64)
    o1 = np.zeros((n, OL.row_bytes(dt, hq * 64)), np.uint8)
    o2 = np.zeros_like(o1)
    oracle.qkv_attn(OL.ptr(q), OL.ptr(k), OL.ptr(v), OL.ptr(o1), dt, hq, hkv, 64, sp, n)
    reference.qkv_attn(OL.ptr(q), OL.ptr(k), OL.ptr(v), OL.ptr(o2), dt, hq, hkv, 64, sp, n)
    assert np.array_equal(o1[sp:], o2[sp:])


@pytest.mark.parametrize("wdt", [Q4, Q8, F16])
def test_token_embed_matches_reference(oracle, reference, wdt):
    rng = np.random.default_rng(wdt)
    table = _rand_w(oracle, rng, wdt, 100, 256)
    adt = F16 if wdt == F16 else Q8
    toks = np.array([5, 99, 0, 5], np.int32)
    o1 = np.zeros((4, OL.row_bytes(adt, 256)), np.uint8)
    o2 = np.zeros_like(o1)
    oracle.token_embed(OL.ptr(table), wdt, OL.ptr(toks), OL.ptr(o1), adt, 256, 100, 0, 4)
    reference.token_embed(OL.ptr(table), wdt, OL.ptr(toks), OL.ptr(o2), adt, 256, 100, 0, 4)
    assert np.array_equal(o1, o2)


# ------------------------------------------------------------------ models --

def _sha(b):
    return hashlib.sha256(np.ascontiguousarray(b).tobytes()).hexdigest()


@pytest.mark.parametrize("name", list(SMALL))
def test_small_models_match_golden(oracle, name):
    w = SMALL[name]
    with open(os.path.join(GOLDEN, f"{name}.json")) as f:
        g = json.load(f)
    cfg = config_of(w)
    prompt = prompt_of(w)
    assert prompt.tolist() == g["prompt"]
    m = oracle.model_create(cfg, w["seed"])
    logits = np.zeros(cfg.n_vocab, np.float32)
    oracle.model_logits(m, OL.ptr(prompt), len(prompt), 0, OL.ptr(logits))
    want = np.load(os.path.join(GOLDEN, f"{name}.prefill_logits.npy"))
    assert np.array_equal(logits.view(np.uint32), want.view(np.uint32))
    adt = F16 if w["wdtype"] == F16 else Q8
    rb = OL.row_bytes(adt, cfg.n_embd)
    for l, digest in enumerate(g["layer_out_sha256"]):
        p = oracle.model_layer_out(m, l, len(prompt) - 1)
        assert _sha(np.ctypeslib.as_array((OL.C.c_uint8 * rb).from_address(p))) == digest, l
    out = np.zeros(w["gen"], np.int32)
    n = oracle.generate_greedy(m, OL.ptr(prompt), len(prompt), w["gen"], OL.ptr(out))
    assert out[:n].tolist() == g["tokens"]
    oracle.model_free(m)


def test_generator_statistics_and_determinism(oracle):
    n = 1 << 20
    a = np.zeros(n, np.float32)
    b = np.zeros(n, np.float32)
    oracle.gen_normal(9, 3, 0.02, n, OL.ptr(a))
    oracle.gen_normal(9, 3, 0.02, n, OL.ptr(b))
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 1e-4 and abs(a.std() - 0.02) < 2e-4
    assert np.abs(a).max() <= 6 * 0.02 + 1e-6  # Irwin-Hall support is [-6, 6] sigma
    t = np.zeros(1000, np.int32)
    oracle.gen_tokens(5, 1000, 32000, OL.ptr(t))
    assert t.min() >= 0 and t.max() < 32000 and len(set(t.tolist())) > 900


def test_argmax_first_max(oracle):
    x = np.array([1.0, 3.0, 2.0, 3.0, -np.inf], np.float32)
    assert oracle.argmax(OL.ptr(x), 5) == 1
