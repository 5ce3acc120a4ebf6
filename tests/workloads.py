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


# Models at the workloads' widths but two or three layers deep: their
# single-row steps run the fused decode kernels (the gate|up kernel is built
# for rows of 2048 and 2304 values), checked against the oracle.
WIDE = {
    "wide-llama-q4": dict(arch=nc.LLAMA, wdtype=nc.Q4, n_vocab=32000, n_embd=2048, n_layers=2, n_heads=32,
                          n_kv_heads=4, n_ffn=5632, eos=-1, rope_pct=1.0, prompt=16, gen=16, seed=0x7EE0001),
    "wide-llama-q8": dict(arch=nc.LLAMA, wdtype=nc.Q8, n_vocab=32000, n_embd=2048, n_layers=2, n_heads=32,
                          n_kv_heads=4, n_ffn=5632, eos=-1, rope_pct=1.0, prompt=16, gen=16, seed=0x7EE0002),
    # MiniCPM's own vocabulary: its tied lm head runs the row-chain kernel
    "wide-minicpm-q4": dict(arch=nc.MINICPM, wdtype=nc.Q4, n_vocab=122753, n_embd=2304, n_layers=2, n_heads=36,
                            n_kv_heads=36, n_ffn=5760, eos=-1, rope_pct=1.0, prompt=16, gen=16, seed=0x7EE0003),
    # the same with its tied embedding scaled by 1/64 (fp16 block deltas;
    # emb_scale): the synthetic embedding otherwise dominates the residual
    # stream, and a tied head then repeats the last prompt token forever; at
    # this scale the greedy stream varies from the fifth step, so the decode
    # graph's next-step embedding (x12, written by the lm head) sees changing
    # tokens
    "wide-minicpm-q4-varied": dict(arch=nc.MINICPM, wdtype=nc.Q4, n_vocab=122753, n_embd=2304, n_layers=2,
                                   n_heads=36, n_kv_heads=36, n_ffn=5760, eos=-1, rope_pct=1.0, prompt=16, gen=16,
                                   seed=0x7EE0003, emb_scale=1.0 / 64),
    # fp16 at MiniCPM's widths: the unrolled fp16 decode matvec for rows of
    # 2304 and 5760 values, its SwiGLU epilogue, and the tied 122753-row head
    "wide-minicpm-f16": dict(arch=nc.MINICPM, wdtype=nc.F16, n_vocab=122753, n_embd=2304, n_layers=2, n_heads=36,
                             n_kv_heads=36, n_ffn=5760, eos=-1, rope_pct=1.0, prompt=16, gen=16, seed=0x7EE0005),
    # TinyLlama's widths in fp16 (the fused rms_norm fp16 decode matvecs at
    # K = 2048) and Zephyr's in Q4 and Q8 (the fused layer_norm with bias on
    # a Q8 row)
    "wide-llama-f16": dict(arch=nc.LLAMA, wdtype=nc.F16, n_vocab=32000, n_embd=2048, n_layers=2, n_heads=32,
                           n_kv_heads=4, n_ffn=5632, eos=-1, rope_pct=1.0, prompt=16, gen=16, seed=0x7EE0006),
    "wide-zephyr-q4": dict(arch=nc.ZEPHYR, wdtype=nc.Q4, n_vocab=100352, n_embd=2048, n_layers=2, n_heads=32,
                           n_kv_heads=32, n_ffn=5632, eos=-1, rope_pct=0.25, prompt=16, gen=16, seed=0x7EE0007),
    "wide-zephyr-q8": dict(arch=nc.ZEPHYR, wdtype=nc.Q8, n_vocab=100352, n_embd=2048, n_layers=2, n_heads=32,
                           n_kv_heads=32, n_ffn=5632, eos=-1, rope_pct=0.25, prompt=16, gen=16, seed=0x7EE0008),
    "wide-openelm-q8": dict(arch=nc.OPENELM, wdtype=nc.Q8, n_vocab=32000, n_embd=2048, n_layers=3,
                            n_heads=[16, 16, 20], n_kv_heads=[4, 4, 5], n_ffn=[1024, 4608, 8192], eos=-1,
                            rope_pct=1.0, prompt=16, gen=16, seed=0x7EE0004),
    # OpenELM sm and md widths (openelm/openelm.h:26-42: 1280 and 1536
    # values), three of their layers' head and FFN widths
    "wide-openelm-sm-q8": dict(arch=nc.OPENELM, wdtype=nc.Q8, n_vocab=32000, n_embd=1280, n_layers=3,
                               n_heads=[12, 16, 20], n_kv_heads=[3, 4, 5], n_ffn=[768, 2816, 5120], eos=-1,
                               rope_pct=1.0, prompt=16, gen=16, seed=0x7EE0009),
    "wide-openelm-md-q4": dict(arch=nc.OPENELM, wdtype=nc.Q4, n_vocab=32000, n_embd=1536, n_layers=3,
                               n_heads=[12, 16, 24], n_kv_heads=[3, 4, 6], n_ffn=[768, 3072, 6144], eos=-1,
                               rope_pct=1.0, prompt=16, gen=16, seed=0x7EE000A),
}

# Long contexts: the reference's default inference context is 1024 positions
# (src/nanochat.cpp:40) and its models allow up to 2048 (TinyLlama, MiniCPM)
# or 4096 (Zephyr).  One-layer models whose prompts fill most of such a
# context; their decode steps cross the 1024-position point where a softmax
# sum changes from one wavefront's loop to the exact workgroup sum.  The
# llama and openelm models run the fused decode kernels (full widths), the
# other two the op-by-op kernels (Q8 and fp16 activations).  Fixtures come
# from the reference build like the others.
LONG = {
    "long-llama-q4": dict(arch=nc.LLAMA, wdtype=nc.Q4, n_vocab=2000, n_embd=2048, n_layers=1, n_heads=32,
                          n_kv_heads=4, n_ffn=256, eos=-1, rope_pct=1.0, prompt=1012, gen=24, seed=0x10C0001),
    "long-openelm-q8": dict(arch=nc.OPENELM, wdtype=nc.Q8, n_vocab=2000, n_embd=2048, n_layers=1, n_heads=[16],
                            n_kv_heads=[4], n_ffn=[512], eos=-1, rope_pct=1.0, prompt=2036, gen=12,
                            seed=0x10C0002),
    "long-minicpm-q8": dict(arch=nc.MINICPM, wdtype=nc.Q8, n_vocab=1000, n_embd=256, n_layers=1, n_heads=4,
                            n_kv_heads=4, n_ffn=512, eos=-1, rope_pct=1.0, prompt=1500, gen=40, seed=0x10C0003),
    "long-zephyr-f16": dict(arch=nc.ZEPHYR, wdtype=nc.F16, n_vocab=1000, n_embd=256, n_layers=1, n_heads=4,
                            n_kv_heads=4, n_ffn=512, eos=-1, rope_pct=0.25, prompt=4080, gen=16, seed=0x10C0004),
}

# The text path (greedy_sample: prompt text -> tokens -> model -> text):
# small models over the synthetic vocabulary of tests/golden/tok/ (482
# pieces, ids up to 511 decode to nothing), the inference context is
# prompt + generated tokens.
CHAT_TOKENIZER = "bpe_chat"
CHAT_PROMPTS = ["Tell me a story about the quick brown fox.", "hello world", "abc " * 12]
CHAT_TOPK = dict(temp=0.9, top_k=50, seed=7)
CHAT = {
    "chat-llama-q8": dict(arch=nc.LLAMA, wdtype=nc.Q8, n_vocab=512, n_embd=256, n_layers=2, n_heads=4,
                          n_kv_heads=2, n_ffn=512, eos=2, rope_pct=1.0, prompt=0, gen=96, seed=2101),
    "chat-minicpm-q4": dict(arch=nc.MINICPM, wdtype=nc.Q4, n_vocab=512, n_embd=256, n_layers=2, n_heads=4,
                            n_kv_heads=4, n_ffn=512, eos=2, rope_pct=1.0, prompt=0, gen=96, seed=2102),
    "chat-zephyr-f16": dict(arch=nc.ZEPHYR, wdtype=nc.F16, n_vocab=512, n_embd=256, n_layers=2, n_heads=4,
                            n_kv_heads=4, n_ffn=512, eos=2, rope_pct=0.25, prompt=0, gen=96, seed=2103),
    "chat-openelm-q8": dict(arch=nc.OPENELM, wdtype=nc.Q8, n_vocab=512, n_embd=256, n_layers=3,
                            n_heads=[2, 2, 3], n_kv_heads=[1, 1, 1], n_ffn=[256, 512, 768], eos=2,
                            rope_pct=1.0, prompt=0, gen=96, seed=2104),
}

ALL = dict(SMALL, **WIDE, **LONG, **nc.WORKLOADS)


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
