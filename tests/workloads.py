"""Model configurations of the tests: small models of every architecture
(fast enough for the oracle) and the full-size workloads of the package."""
import numpy as np

import oracle_lib as OL
from nc_pkg import nc

SMALL = {
    "small-llama-q4": dict(arch=nc.LLAMA, wdtype=nc.Q4, n_vocab=1000, n_embd=256, n_layers=2, n_heads=4,
                           n_kv_heads=2, n_ffn=512, eos=-1, rope_pct=1.0, prompt=16, gen=32, seed=1234),
    "small-llama-q8": dict(arch=nc.LLAMA, wdtype=nc.Q8, n_vocab=1000, n_embd=256, n_layers=2, n_heads=4,
                           n_kv_heads=1, n_ffn=512, eos=-1, rope_pct=1.0, prompt=16, gen=32, seed=1235),
    "small-llama-f16": dict(arch=nc.LLAMA, wdtype=nc.F16, n_vocab=1000, n_embd=256, n_layers=2, n_heads=4,
                            n_kv_heads=2, n_ffn=512, eos=-1, rope_pct=1.0, prompt=16, gen=32, seed=1236),
    "small-zephyr-f16": dict(arch=nc.ZEPHYR, wdtype=nc.F16, n_vocab=1000, n_embd=256, n_layers=2, n_heads=4,
                             n_kv_heads=4, n_ffn=512, eos=999, rope_pct=0.25, prompt=16, gen=32, seed=1237),
    "small-minicpm-q4": dict(arch=nc.MINICPM, wdtype=nc.Q4, n_vocab=1000, n_embd=256, n_layers=2, n_heads=4,
                             n_kv_heads=4, n_ffn=512, eos=2, rope_pct=1.0, prompt=16, gen=32, seed=1238),
    "small-openelm-q8": dict(arch=nc.OPENELM, wdtype=nc.Q8, n_vocab=1000, n_embd=256, n_layers=3,
                             n_heads=[2, 2, 3], n_kv_heads=[1, 1, 1], n_ffn=[256, 512, 768], eos=-1,
                             rope_pct=1.0, prompt=16, gen=32, seed=1239),
    # the model x dtype combinations the full-size workloads do not cover
    "small-zephyr-q8": dict(arch=nc.ZEPHYR, wdtype=nc.Q8, n_vocab=1000, n_embd=256, n_layers=2, n_heads=4,
                            n_kv_heads=4, n_ffn=512, eos=999, rope_pct=0.25, prompt=16, gen=32, seed=1240),
    "small-zephyr-q4": dict(arch=nc.ZEPHYR, wdtype=nc.Q4, n_vocab=1000, n_embd=256, n_layers=2, n_heads=4,
                            n_kv_heads=4, n_ffn=512, eos=999, rope_pct=0.25, prompt=16, gen=32, seed=1241),
    "small-minicpm-f16": dict(arch=nc.MINICPM, wdtype=nc.F16, n_vocab=1000, n_embd=256, n_layers=2, n_heads=4,
                              n_kv_heads=4, n_ffn=512, eos=2, rope_pct=1.0, prompt=16, gen=32, seed=1242),
    "small-minicpm-q8": dict(arch=nc.MINICPM, wdtype=nc.Q8, n_vocab=1000, n_embd=256, n_layers=2, n_heads=4,
                             n_kv_heads=4, n_ffn=512, eos=2, rope_pct=1.0, prompt=16, gen=32, seed=1243),
    "small-openelm-f16": dict(arch=nc.OPENELM, wdtype=nc.F16, n_vocab=1000, n_embd=256, n_layers=3,
                              n_heads=[2, 2, 3], n_kv_heads=[1, 1, 1], n_ffn=[256, 512, 768], eos=-1,
                              rope_pct=1.0, prompt=16, gen=32, seed=1244),
}


ALL = dict(SMALL, **nc.WORKLOADS)


def config_of(w, cls=OL.Config, max_ctx=None):
    """or_config / nc_model_config of a workload dict (same field layout)."""
    return nc.make_config(w["arch"], w["wdtype"], w["n_vocab"], w["n_embd"], w["n_layers"], w["n_heads"],
                          w["n_kv_heads"], w["n_ffn"], max_ctx or (w["prompt"] + w["gen"]), eos=w["eos"],
                          rope_pct=w["rope_pct"], cls=cls)


def prompt_of(w):
    """The workload's prompt: token ids uniform in [0, vocab) from its seed."""
    p = np.zeros(w["prompt"], np.int32)
    OL.Oracle().gen_tokens(w["seed"] + nc.PROMPT_SEED_OFFSET, w["prompt"], w["n_vocab"], OL.ptr(p))
    return p
