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
        x[: max(1, n // 100)] = 400.0
    else:
        raise ValueError(kind)
    return np.ascontiguousarray(x, np.float32)


KINDS = ["normal", "ties", "flat", "two_level", "signed_zero", "peaked", "overflow"]


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
