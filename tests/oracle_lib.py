"""ctypes bindings for the checker libraries (test infrastructure).

* ``oracle/_build/liboracle.so``: the C restatement of the reference numerics.
* ``oracle/_ref/libgten_ref.so``: the reference's own gten sources plus a
  harness (built only where the reference source tree exists).

Only tests, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline load
these; the product path never does.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "_build", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libgten_ref.so")
# the reference source tree (build container only): its tokenizer vocabularies
REFERENCE_ROOT = os.environ.get("NC_REFERENCE_ROOT", "/root/reference")

I32, F16, F32, Q8, Q4 = 0, 1, 2, 3, 4
LLAMA, ZEPHYR, MINICPM, OPENELM = 0, 1, 2, 3
MAX_LAYERS = 64
W_SLOTS = ["Q", "K", "V", "O", "GATE", "UP", "DOWN", "ATTN_NORM", "ATTN_NORM_B", "MLP_NORM",
           "MLP_NORM_B", "Q_BIAS", "K_BIAS", "V_BIAS", "Q_NORM", "K_NORM"]
TID_EMB, TID_NORM, TID_NORM_B, TID_LM = 0xFFFF0, 0xFFFF1, 0xFFFF2, 0xFFFF3


class Config(C.Structure):
    _fields_ = [("arch", C.c_int), ("wdtype", C.c_int), ("n_vocab", C.c_int), ("n_embd", C.c_int),
                ("n_layers", C.c_int), ("d_head", C.c_int), ("max_ctx", C.c_int), ("eos", C.c_int),
                ("rope_pct", C.c_float), ("n_heads", C.c_int * MAX_LAYERS),
                ("n_kv_heads", C.c_int * MAX_LAYERS), ("n_ffn", C.c_int * MAX_LAYERS)]


def make_config(arch, wdtype, n_vocab, n_embd, n_layers, n_heads, n_kv_heads, n_ffn, max_ctx,
                eos=-1, rope_pct=1.0, d_head=64):
    c = Config()
    c.arch, c.wdtype, c.n_vocab, c.n_embd, c.n_layers = arch, wdtype, n_vocab, n_embd, n_layers
    c.d_head, c.max_ctx, c.eos, c.rope_pct = d_head, max_ctx, eos, rope_pct
    as_list = lambda v: list(v) if isinstance(v, (list, tuple)) else [v] * n_layers
    for i, (h, kv, f) in enumerate(zip(as_list(n_heads), as_list(n_kv_heads), as_list(n_ffn))):
        c.n_heads[i], c.n_kv_heads[i], c.n_ffn[i] = h, kv, f
    return c


def row_bytes(dt, cols):
    if dt == Q8:
        return (cols + 31) // 32 * 34
    if dt == Q4:
        return cols // 32 * 18
    if dt == F16:
        return cols * 2
    return cols * 4


def ptr(a):
    return a.ctypes.data_as(C.c_void_p)


_VP, _I, _F, _U64 = C.c_void_p, C.c_int, C.c_float, C.c_uint64


def _bind(lib, name, res, args):
    f = getattr(lib, name)
    f.restype, f.argtypes = res, args
    return f


class _Lib:
    """Common op surface of the oracle (prefix ``or_``) and the reference harness
    (prefix ``ref_``); both take the reference's byte layouts."""

    def __init__(self, path, prefix):
        self.lib = C.CDLL(path)
        p = prefix
        b = lambda n, r, a: _bind(self.lib, p + n, r, a)
        self.fp16_to_fp32 = b("fp16_to_fp32", _F, [C.c_uint16])
        self.fp32_to_fp16 = b("fp32_to_fp16", C.c_uint16, [_F])
        self.q8_quantize_row = b("q8_quantize_row", None, [_VP, _VP, _I])
        self.matmul = b("matmul", None, [_VP, _I, _VP, _I, _VP, _I, _I, _I, _I, _I] + ([_VP] if p == "or_" else []))
        self.rms_norm = b("rms_norm", None, [_VP, _I, _VP, _VP, _I, _I, _I])
        self.rms_norm_heads = b("rms_norm_heads", None, [_VP, _I, _VP, _VP, _I, _I, _I, _I])
        self.layer_norm = b("layer_norm", None, [_VP, _I, _VP, _VP, _VP, _I, _I, _I])
        self.rotary_emb = b("rotary_emb", None, [_VP, _VP, _I, _I, _I, _F, _I, _I])
        self.silu = b("silu", None, [_VP, _VP, _I, _I, _I, _I])
        self.multiply = b("multiply", None, [_VP, _VP, _VP, _I, _I, _I, _I])
        self.add = b("add", None, [_VP, _VP, _VP, _I, _I, _I, _I])
        self.scale = b("scale", None, [_VP, _I, _F, _I, _I, _I])
        self.bias_add = b("bias_add", None, [_VP, _I, _VP, _I, _I, _I])
        self.qkv_attn = b("qkv_attn", None, [_VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I])
        self.generate_greedy = b("generate_greedy", _I, [_VP, _VP, _I, _I, _VP])
        self.model_logits = b("model_logits", None, [_VP, _VP, _I, _I, _VP])
        self.model_layer_out = b("model_layer_out", _VP, [_VP, _I, _I])
        self.model_free = b("model_free", None, [_VP])


class Oracle(_Lib):
    def __init__(self):
        super().__init__(ORACLE_SO, "or_")
        b = lambda n, r, a: _bind(self.lib, n, r, a)
        self.token_embed_ = b("or_token_embed", None, [_VP, _I, _VP, _VP, _I, _I, _I, _I])
        self.q8_quantize_weights = b("or_q8_quantize_weights", None, [_VP, C.c_int64, _VP])
        self.q4_quantize_weights = b("or_q4_quantize_weights", None, [_VP, C.c_int64, _VP])
        self.gen_normal = b("or_gen_normal", None, [_U64, C.c_uint32, _F, C.c_int64, _VP])
        self.gen_tokens = b("or_gen_tokens", None, [_U64, _I, _I, _VP])
        self.dot = b("or_dot", _F, [_VP, _I, _VP, _I, _I])
        self.read_row = b("or_read_row", None, [_VP, _I, _VP, _I])
        self.seq_sum = b("or_seq_sum", _F, [_VP, _I])
        self.expf = b("or_expf", _F, [_F])
        self.argmax = b("or_argmax", _I, [_VP, _I])
        self.model_create_ = b("or_model_create", _VP, [C.POINTER(Config)])
        self.model_init_synthetic = b("or_model_init_synthetic", None, [_VP, _U64])
        self.model_weight = b("or_model_weight", _VP, [_VP, _I, _I])
        self.make_weight = b("or_make_weight", None, [C.POINTER(Config), _U64, _I, _I, _VP])
        self.weight_shape_ = b("or_weight_shape", _I, [C.POINTER(Config), _I, _I, C.POINTER(_I), C.POINTER(_I),
                                                        C.POINTER(_I)])

        self.mt_seed = b("or_mt_seed", None, [C.c_uint32, _VP])
        self.mt_next = b("or_mt_next", C.c_uint32, [_VP])
        self.mt_canonical = b("or_mt_canonical", C.c_double, [_VP])
        self.topk_sample = b("or_topk_sample", _I, [_VP, _I, _F, _I, _VP, _VP])
        self.exp = b("or_exp", C.c_double, [C.c_double])
        self.exp_probe_inputs = b("or_exp_probe_inputs", None, [_U64, C.c_int64, C.c_int64, _VP])
        self.check_exp_fn = b("or_check_exp_fn", C.c_int64, [_VP, _U64, C.c_int64, C.POINTER(C.c_double)])
        self.exp_mismatches = b("or_exp_mismatches", C.c_int64, [_VP, _VP, C.c_int64, C.POINTER(C.c_int64)])
        self.generate_topk = b("or_generate_topk", _I, [_VP, _VP, _I, _I, _F, _I, C.c_uint32, _VP])

    def token_embed(self, table, wdt, tokens, out, adt, d, vocab, start, n_ctx):
        self.token_embed_(table, wdt, tokens, out, adt, d, start, n_ctx)

    def model_create(self, cfg, seed):
        m = self.model_create_(C.byref(cfg))
        self.model_init_synthetic(m, seed)
        return m

    def weight_shape(self, cfg, layer, slot):
        r, c, d = _I(), _I(), _I()
        ok = self.weight_shape_(C.byref(cfg), layer, slot, C.byref(r), C.byref(c), C.byref(d))
        return (r.value, c.value, d.value) if ok else None


class Reference(_Lib):
    def __init__(self):
        super().__init__(REF_SO, "ref_")
        b = lambda n, r, a: _bind(self.lib, n, r, a)
        self.token_embed_ = b("ref_token_embed", None, [_VP, _I, _VP, _VP, _I, _I, _I, _I, _I])
        self.model_create_ = b("ref_model_create", _VP, [C.POINTER(Config), _U64])
        self.model_load_gten = b("ref_model_load_gten", _I, [_VP, C.c_char_p])
        self.rng_create = b("ref_rng_create", _VP, [C.c_uint32])
        self.rng_free = b("ref_rng_free", None, [_VP])
        self.rng_next = b("ref_rng_next", C.c_uint32, [_VP])
        self.topk_sample = b("ref_topk_sample", _I, [_VP, _VP, _I, _F, _I, _VP])
        self.generate_topk = b("ref_generate_topk", _I, [_VP, _VP, _I, _I, _F, _I, C.c_uint32, _VP])
        self.tok_llama_create = b("ref_tok_llama_create", _VP, [C.c_char_p, _I, _I, C.c_char_p, C.c_char_p, _VP, _I,
                                                                 _VP, _I])
        self.tok_gpt2_create = b("ref_tok_gpt2_create", _VP, [C.c_char_p, _I, _I])
        self.tok_encode = b("ref_tok_encode", _I, [_VP, C.c_char_p, _VP, _I])
        self.tok_decode = b("ref_tok_decode", C.c_char_p, [_VP, _I, _I])
        self.tok_free = b("ref_tok_free", None, [_VP])
        self.greedy_sample_text_ = b("ref_greedy_sample_text", _I, [_VP, _VP, C.c_char_p, _I, _I, C.c_char_p, _I])

    def greedy_sample_text(self, model, tok, prompt, inference_ctx, train_ctx):
        """gten::greedy_sample's output text (bytes) for a prompt (bytes)."""
        cap = 1 << 16
        buf = C.create_string_buffer(cap)
        n = self.greedy_sample_text_(model, tok, prompt, inference_ctx, train_ctx, buf, cap)
        assert n <= cap
        return buf.raw[:n]

    def token_embed(self, table, wdt, tokens, out, adt, d, vocab, start, n_ctx):
        self.token_embed_(table, wdt, tokens, out, adt, d, vocab, start, n_ctx)

    def model_create(self, cfg, seed):
        return self.model_create_(C.byref(cfg), seed)


def have_reference():
    return os.path.exists(REF_SO)
