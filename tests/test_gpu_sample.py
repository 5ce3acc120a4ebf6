"""Top-k / temperature sampling on the device (nc_sample_topk,
nc_model_generate_topk) against the oracle and the reference's sampled
streams (gten/sampler.cpp:63-143 with std::mt19937(seed)).

* The device exp equals the host glibc exp (std::exp on double) on 16M
  inputs and the edge values.
* One sampling step: the token, the n normalized weights (bit for bit) and
  the generator state after 12 draws equal the oracle's, on every logits
  case of the CPU tests (ties at the k-th value, flat rows, +-0, NaN,
  overflowing exps, clamped top_k and temp), which also drives the exact
  heap-select fallback.
* Model level: the sampled streams of the small models of every family and
  of TinyLlama-Q4 and MiniCPM-Q4 equal the reference harness's fixtures,
  through the graph-replayed step and through direct launches.
"""
import os

import numpy as np
import pytest

import oracle_lib as OL
from test_sample import CASES, golden_topk, logits_case, case_seed
from workloads import ALL, SMALL, config_of, prompt_of

pytestmark = pytest.mark.gpu


def test_device_exp_equals_host_libm(gpu, oracle):
    n = 1 << 24
    x = np.zeros(n, np.float64)
    oracle.exp_probe_inputs(20241203, 0, n, OL.ptr(x))
    edge = [0.0, -0.0, 1e-300, -1e-300, 2.0**-54, 709.782712893384, 709.7827128933841, -708.3964185322641,
            -745.1332191019411, -745.1332191019412, 512.0, -512.0, 1024.0, np.inf, -np.inf, np.nan]
    x[: len(edge)] = edge
    dx, dy = gpu.DeviceBuffer(x.nbytes), gpu.DeviceBuffer(x.nbytes)
    dx.upload(x)
    gpu.check(gpu.lib().nc_exp(OL.C.c_void_p(dx.ptr), OL.C.c_void_p(dy.ptr), n, None), "exp")
    y = dy.download(np.zeros(n, np.float64))
    first = OL.C.c_int64()
    bad = oracle.exp_mismatches(OL.ptr(x), OL.ptr(y), n, OL.C.byref(first))
    assert bad == 0, f"{bad} differ, first x = {x[first.value]!r}"


def run_draws(gpu, oracle, x, k, temp, seed, draws=12):
    n = len(x)
    L = gpu.lib()
    st = np.zeros(625, np.uint32)
    L.nc_rng_seed(seed, OL.ptr(st))
    d_x, d_st = gpu.DeviceBuffer(x.nbytes), gpu.DeviceBuffer(st.nbytes)
    d_tok, d_p = gpu.DeviceBuffer(4), gpu.DeviceBuffer(8 * n)
    d_x.upload(x)
    d_st.upload(st)
    o_st = np.zeros(625, np.uint32)
    oracle.mt_seed(seed, OL.ptr(o_st))
    po = np.zeros(n)
    for draw in range(draws):
        gpu.check(L.nc_sample_topk(OL.C.c_void_p(d_x.ptr), n, temp, k, OL.C.c_void_p(d_st.ptr),
                                   OL.C.c_void_p(d_tok.ptr), OL.C.c_void_p(d_p.ptr), None), "sample_topk")
        tok = int(d_tok.download(np.zeros(1, np.int32))[0])
        pd = d_p.download(np.zeros(n))
        to = oracle.topk_sample(OL.ptr(x), n, temp, k, OL.ptr(o_st), OL.ptr(po))
        assert tok == to, (draw, tok, to)
        same = (pd.view(np.uint64) == po.view(np.uint64)) | (np.isnan(pd) & np.isnan(po))
        assert same.all(), (draw, int(np.argmin(same)))
    assert np.array_equal(d_st.download(np.zeros(625, np.uint32)), o_st)


@pytest.mark.parametrize("kind,n,k,temp", CASES)
def test_sample_topk_matches_oracle(gpu, oracle, kind, n, k, temp):
    x = logits_case(kind, n, seed=case_seed(kind, n, k))
    run_draws(gpu, oracle, x, k, temp, seed=1000 + n + k)


def test_sample_topk_vocab_sizes_and_twist(gpu, oracle):
    """MiniCPM's vocabulary (122753) and Zephyr's (100352); 330 draws cross
    the generator's 624-word regeneration."""
    for n, k in ((122753, 40), (100352, 1000)):
        x = logits_case("normal", n, seed=n)
        run_draws(gpu, oracle, x, k, 0.9, seed=n, draws=4)
    x = logits_case("normal", 32000, seed=5)
    run_draws(gpu, oracle, x, 40, 1.0, seed=5, draws=330)


def test_sample_topk_rejects_bad_arguments(gpu):
    L = gpu.lib()
    d_x, d_st, d_tok = gpu.DeviceBuffer(4 * 100), gpu.DeviceBuffer(4 * 625), gpu.DeviceBuffer(4)
    args = lambda temp, k, n=100: (OL.C.c_void_p(d_x.ptr), n, temp, k, OL.C.c_void_p(d_st.ptr),
                                   OL.C.c_void_p(d_tok.ptr), None, None)
    for temp, k, n in ((1.0, 0, 100), (1.0, 101, 100), (0.0, 5, 100), (-1.0, 5, 100), (float("nan"), 5, 100),
                       (1.0, 1, 1)):
        assert L.nc_sample_topk(*args(temp, k, n)) != 0, (temp, k, n)


def model_runs(gpu, name, n_gen=None):
    w = ALL[name]
    g = golden_topk(name)
    prompt = prompt_of(w)
    assert prompt.tolist() == g["prompt"]
    m = gpu.Model(config_of(w, cls=gpu.ModelConfig))
    m.init_synthetic(w["seed"])
    try:
        for r in g["runs"]:
            toks = m.generate_topk(prompt, r["n_gen"], r["temp"], r["top_k"], r["seed"])
            ref = r["tokens"]
            diff = next((i for i, (a, b) in enumerate(zip(toks.tolist(), ref)) if a != b), None)
            assert toks.tolist() == ref, (r["temp"], r["top_k"], r["seed"], f"first difference at step {diff}")
    finally:
        m.close()


@pytest.mark.parametrize("name", sorted(SMALL))
def test_generate_topk_small_models(gpu, name):
    model_runs(gpu, name)


@pytest.mark.parametrize("name", sorted(SMALL)[:3])
def test_generate_topk_direct_launches(gpu, name, monkeypatch):
    monkeypatch.setenv("NC_DECODE_GRAPH", "0")
    model_runs(gpu, name)


@pytest.mark.parametrize("name", ["tinyllama-q4", "minicpm-q4"])
def test_generate_topk_full_workloads(gpu, name):
    model_runs(gpu, name)
