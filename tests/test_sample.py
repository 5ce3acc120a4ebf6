"""Top-k / temperature sampling (gten/sampler.cpp:63-143) with a seeded
std::mt19937 in place of std::random_device.

CPU: the oracle's restatement (oracle/oracle_sample.c) against the reference
harness, which runs the reference's standard library calls (std::partial_sort,
std::exp, std::discrete_distribution, std::mt19937 from libstdc++): tokens,
the normalized weights and the generator state after the draws, on logits
with and without ties at the k-th value, flat rows, +-0, overflowing exps and
the clamps of top_k and temp.  The generator is pinned by the C++ standard's
known answer (the 10000th output of a default-seeded mt19937 is 4123659995).
"""
import numpy as np
import pytest

import oracle_lib as OL


def logits_case(kind, n, seed):
    rng = np.random.default_rng(seed)
    if kind == "normal":
        x = rng.normal(0.0, 3.0, n)
    elif kind == "ties":  # a quarter-step grid: many equal values at every rank
        x = np.round(rng.normal(0.0, 3.0, n) * 4) / 4
    elif kind == "flat":
        x = np.zeros(n)
    elif kind == "two_level":
        x = np.where(rng.random(n) < 0.01, 5.0, -5.0)
    elif kind == "signed_zero":
        x = np.where(rng.random(n) < 0.5, 0.0, -0.0)
        x[rng.random(n) < 0.002] = 1.0
    elif kind == "peaked":
        x = rng.normal(0.0, 1.0, n)
        x[rng.integers(n)] = 40.0
    elif kind == "overflow":  # exp(x / temp) overflows: infinite sum, NaN weights
        x = rng.normal(0.0, 3.0, n)
        x[: max(1, n // 100)] = 1500.0
    elif kind == "overflow_late":  # as above, the overflowing logits last: token 0 is drawn, unkept
        x = rng.normal(0.0, 3.0, n)
        x[-max(1, n // 100):] = 1500.0
    elif kind == "nan":  # a NaN logit never compares greater: the heap order keeps or drops it
        x = rng.normal(0.0, 3.0, n)
        x[rng.integers(n)] = np.nan
    else:
        raise ValueError(kind)
    return np.ascontiguousarray(x, np.float32)


KINDS = ["normal", "ties", "flat", "two_level", "signed_zero", "peaked", "overflow", "overflow_late", "nan"]


def case_seed(kind, n, k):
    return KINDS.index(kind) * 1000003 + n * 7 + k


CASES = [(kind, n, k, t) for kind in KINDS for n, k, t in
         [(2, 1, 1.0), (5, 3, 0.7), (1000, 40, 1.0), (1000, 1000, 0.5), (32000, 1, 1.0), (32000, 40, 0.8),
          (32000, 1000, 1.0), (32000, 5000, 3.0)]]


def same_bits(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.array_equal(a.view(np.uint64), b.view(np.uint64)) or \
        bool(np.all((a.view(np.uint64) == b.view(np.uint64)) | (np.isnan(a) & np.isnan(b))))


def test_mt19937_known_answer_and_reference(oracle, reference):
    st = np.zeros(625, np.uint32)
    oracle.mt_seed(5489, OL.ptr(st))
    outs = [oracle.mt_next(OL.ptr(st)) for _ in range(10000)]
    assert outs[-1] == 4123659995  # [rand.predef]
    for seed in (0, 1, 0xFFFFFFFF, 123456789):
        oracle.mt_seed(seed, OL.ptr(st))
        g = reference.rng_create(seed)
        a = [oracle.mt_next(OL.ptr(st)) for _ in range(1500)]
        b = [reference.rng_next(g) for _ in range(1500)]
        reference.rng_free(g)
        assert a == b, seed


def test_mt19937_known_answer_without_reference(oracle):
    st = np.zeros(625, np.uint32)
    oracle.mt_seed(5489, OL.ptr(st))
    for _ in range(9999):
        oracle.mt_next(OL.ptr(st))
    assert oracle.mt_next(OL.ptr(st)) == 4123659995


@pytest.mark.parametrize("kind,n,k,temp", CASES)
def test_topk_sample_matches_reference(oracle, reference, kind, n, k, temp):
    x = logits_case(kind, n, seed=case_seed(kind, n, k))
    seed = 1000 + n + k
    st = np.zeros(625, np.uint32)
    oracle.mt_seed(seed, OL.ptr(st))
    g = reference.rng_create(seed)
    po, pr = np.zeros(n), np.zeros(n)
    try:
        for draw in range(12):
            to = oracle.topk_sample(OL.ptr(x), n, temp, k, OL.ptr(st), OL.ptr(po))
            tr = reference.topk_sample(g, OL.ptr(x), n, temp, k, OL.ptr(pr))
            assert to == tr, (draw, to, tr)
            assert same_bits(po, pr), draw
        assert oracle.mt_next(OL.ptr(st)) == reference.rng_next(g)
    finally:
        reference.rng_free(g)


def test_tie_cases_exercise_the_heap_order(reference):
    """At least one tie case keeps a set of tied indices that a stable
    top-k (lowest indices first) would not: the cases above check the
    reference's heap order, not just any tie rule."""
    differs = 0
    for kind in ("ties", "flat", "two_level", "signed_zero"):
        for n, k in ((1000, 40), (32000, 40), (32000, 1000)):
            x = logits_case(kind, n, seed=case_seed(kind, n, k))
            g = reference.rng_create(7)
            pr = np.zeros(n)
            reference.topk_sample(g, OL.ptr(x), n, 1.0, k, OL.ptr(pr))
            reference.rng_free(g)
            stable = set(np.argsort(-x.astype(np.float64), kind="stable")[:k].tolist())
            differs += set(np.nonzero(pr)[0].tolist()) != stable
    assert differs > 0


def test_kernel_exp_equals_host_libm(nc, oracle):
    """The kernels' double exp (evaluated on the host from the same source)
    equals the host glibc exp -- std::exp on double, the reference's -- on
    10^8 inputs: the full bit-pattern range, [-750, 710] and [-40, 40]."""
    fn = OL.C.cast(nc.lib().nc_exp_host, OL.C.c_void_p).value
    first = OL.C.c_double()
    bad = oracle.check_exp_fn(fn, 20241202, 100_000_000, OL.C.byref(first))
    assert bad == 0, f"{bad} inputs differ, first x = {first.value!r}"
    for x in [0.0, -0.0, 1e-300, -1e-300, 2.0**-54, 709.782712893384, 709.7827128933841, -708.3964185322641,
              -745.1332191019411, -745.1332191019412, 512.0, -512.0, 1024.0, float("inf"), float("-inf"),
              float("nan")]:
        a, b = nc.lib().nc_exp_host(x), oracle.exp(x)
        assert np.float64(a).view(np.uint64) == np.float64(b).view(np.uint64) or (np.isnan(a) and np.isnan(b)), x


def test_rng_seed_matches_oracle(nc, oracle):
    for seed in (0, 5489, 0xFFFFFFFF):
        a, b = np.zeros(625, np.uint32), np.zeros(625, np.uint32)
        assert nc.lib().nc_rng_seed(seed, OL.ptr(a)) == 0
        oracle.mt_seed(seed, OL.ptr(b))
        assert np.array_equal(a, b)


def golden_topk(name):
    import json
    import os
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", f"{name}.topk.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("name", sorted(__import__("workloads").SMALL))
def test_oracle_topk_streams_match_reference_fixtures(oracle, name):
    """The oracle's model with the oracle's sampler gives the reference's
    sampled streams (tests/golden/*.topk.json, from the reference harness)."""
    from workloads import SMALL, config_of, prompt_of
    w = SMALL[name]
    g = golden_topk(name)
    cfg = config_of(w)
    prompt = prompt_of(w)
    assert prompt.tolist() == g["prompt"]
    for r in g["runs"]:
        m = oracle.model_create(cfg, w["seed"])
        out = np.zeros(r["n_gen"], np.int32)
        n = oracle.generate_topk(m, OL.ptr(prompt), len(prompt), r["n_gen"], r["temp"], r["top_k"], r["seed"],
                                 OL.ptr(out))
        oracle.model_free(m)
        assert out[:n].tolist() == r["tokens"], r
