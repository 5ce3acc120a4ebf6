"""MI355X (gfx950) decode path of nanochatllms.cpp behind a C-ABI.

The product is ``_build/libgten_hip.so`` (HIP kernels + C entry points declared
in ``include/gten_hip.h``).  This module is the Python host mirror used by the
tests and the benchmark: ctypes bindings, device tensors, and the model
workloads.  It never falls back to a CPU path: if the library is missing or
the GPU is unavailable, calls raise.

The directory name contains a dot, so import it with :func:`load_package`
from a file path, e.g. ``importlib`` with ``spec_from_file_location``.
"""
import ctypes as C
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "_build", "libgten_hip.so")

I32, F16, F32, Q8, Q4 = 0, 1, 2, 3, 4
LLAMA, ZEPHYR, MINICPM, OPENELM = 0, 1, 2, 3
MAX_LAYERS = 64
W_Q, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN = range(7)
W_ATTN_NORM, W_ATTN_NORM_B, W_MLP_NORM, W_MLP_NORM_B = 7, 8, 9, 10
W_Q_BIAS, W_K_BIAS, W_V_BIAS, W_Q_NORM, W_K_NORM = 11, 12, 13, 14, 15
TID_EMB, TID_NORM, TID_NORM_B, TID_LM = 0xFFFF0, 0xFFFF1, 0xFFFF2, 0xFFFF3
MAX_CTX = 4096  # NC_MAX_CTX


class HipError(RuntimeError):
    pass


class Tensor(C.Structure):
    """nc_tensor: a device tensor descriptor (no ownership)."""
    _fields_ = [("data", C.c_void_p), ("deltas", C.c_void_p), ("dtype", C.c_int), ("rows", C.c_int),
                ("cols", C.c_int), ("pitch", C.c_int)]


class ModelConfig(C.Structure):
    """nc_model_config (field layout shared with the oracle's or_config)."""
    _fields_ = [("arch", C.c_int), ("wdtype", C.c_int), ("n_vocab", C.c_int), ("n_embd", C.c_int),
                ("n_layers", C.c_int), ("d_head", C.c_int), ("max_ctx", C.c_int), ("eos", C.c_int),
                ("rope_pct", C.c_float), ("n_heads", C.c_int * MAX_LAYERS),
                ("n_kv_heads", C.c_int * MAX_LAYERS), ("n_ffn", C.c_int * MAX_LAYERS)]


def make_config(arch, wdtype, n_vocab, n_embd, n_layers, n_heads, n_kv_heads, n_ffn, max_ctx, eos=-1,
                rope_pct=1.0, d_head=64, cls=ModelConfig):
    c = cls()
    c.arch, c.wdtype, c.n_vocab, c.n_embd, c.n_layers = arch, wdtype, n_vocab, n_embd, n_layers
    c.d_head, c.max_ctx, c.eos, c.rope_pct = d_head, max_ctx, eos, rope_pct
    as_list = lambda v: list(v) if isinstance(v, (list, tuple)) else [v] * n_layers
    for i, (h, kv, f) in enumerate(zip(as_list(n_heads), as_list(n_kv_heads), as_list(n_ffn))):
        c.n_heads[i], c.n_kv_heads[i], c.n_ffn[i] = h, kv, f
    return c


# The five workloads: model shapes of the reference's configs
# (tinyllama/tinyllama.h:12-24 with vocab 32000, zephyr/zephyr.h:10-23,
# minicpm/minicpm.h:9-24, an OpenELM-1.1B-like ramp on openelm/openelm.h:13-24),
# synthetic N(0, 0.02) weights, random prompts of `prompt` tokens and `gen`
# greedy tokens; max_ctx = prompt + gen.
_ELM_F = [1024, 1280, 1536, 1792, 2048, 2304, 2560, 2816, 3072, 3328, 3584, 3840, 4096, 4608, 4608, 5120,
          5376, 5632, 5888, 6144, 6400, 6656, 6912, 7168, 7424, 7680, 7936, 8192]
WORKLOADS = {
    "tinyllama-q8": dict(arch=LLAMA, wdtype=Q8, n_vocab=32000, n_embd=2048, n_layers=22, n_heads=32, n_kv_heads=4,
                         n_ffn=5632, eos=32002, rope_pct=1.0, prompt=64, gen=128, seed=0x5EED0001),
    "tinyllama-q4": dict(arch=LLAMA, wdtype=Q4, n_vocab=32000, n_embd=2048, n_layers=22, n_heads=32, n_kv_heads=4,
                         n_ffn=5632, eos=32002, rope_pct=1.0, prompt=64, gen=256, seed=0x5EED0001),
    "zephyr-f16": dict(arch=ZEPHYR, wdtype=F16, n_vocab=100352, n_embd=2048, n_layers=24, n_heads=32,
                       n_kv_heads=32, n_ffn=5632, eos=100257, rope_pct=0.25, prompt=128, gen=128, seed=0x5EED0003),
    "minicpm-q4": dict(arch=MINICPM, wdtype=Q4, n_vocab=122753, n_embd=2304, n_layers=40, n_heads=36,
                       n_kv_heads=36, n_ffn=5760, eos=2, rope_pct=1.0, prompt=512, gen=128, seed=0x5EED0004),
    "openelm-q8": dict(arch=OPENELM, wdtype=Q8, n_vocab=32000, n_embd=2048, n_layers=28,
                       n_heads=[16] * 12 + [20] * 16, n_kv_heads=[4] * 12 + [5] * 16, n_ffn=_ELM_F,
                       eos=32002, rope_pct=1.0, prompt=64, gen=256, seed=0x5EED0005),
    # the reference's other published rows (README.md:36-44) at full size
    "tinyllama-f16": dict(arch=LLAMA, wdtype=F16, n_vocab=32000, n_embd=2048, n_layers=22, n_heads=32,
                          n_kv_heads=4, n_ffn=5632, eos=32002, rope_pct=1.0, prompt=64, gen=128, seed=0x5EED0001),
    "zephyr-q4": dict(arch=ZEPHYR, wdtype=Q4, n_vocab=100352, n_embd=2048, n_layers=24, n_heads=32,
                      n_kv_heads=32, n_ffn=5632, eos=100257, rope_pct=0.25, prompt=128, gen=128, seed=0x5EED0003),
    "zephyr-q8": dict(arch=ZEPHYR, wdtype=Q8, n_vocab=100352, n_embd=2048, n_layers=24, n_heads=32,
                      n_kv_heads=32, n_ffn=5632, eos=100257, rope_pct=0.25, prompt=128, gen=128, seed=0x5EED0003),
    "minicpm-q8": dict(arch=MINICPM, wdtype=Q8, n_vocab=122753, n_embd=2304, n_layers=40, n_heads=36,
                       n_kv_heads=36, n_ffn=5760, eos=2, rope_pct=1.0, prompt=64, gen=128, seed=0x5EED0004),
    "minicpm-f16": dict(arch=MINICPM, wdtype=F16, n_vocab=122753, n_embd=2304, n_layers=40, n_heads=36,
                        n_kv_heads=36, n_ffn=5760, eos=2, rope_pct=1.0, prompt=64, gen=128, seed=0x5EED0004),
    # OpenELM's sm and md configurations (openelm/openelm.h:26-42) in Q8
    "openelm-sm-q8": dict(arch=OPENELM, wdtype=Q8, n_vocab=32000, n_embd=1280, n_layers=16,
                          n_heads=[12] * 5 + [16] * 7 + [20] * 4, n_kv_heads=[3] * 5 + [4] * 7 + [5] * 4,
                          n_ffn=[768, 1024, 1280, 1536, 1792, 2048, 2560, 2816, 3072, 3328, 3584, 3840, 4352, 4608,
                                 4864, 5120],
                          eos=32002, rope_pct=1.0, prompt=64, gen=128, seed=0x5EED0006),
    "openelm-md-q8": dict(arch=OPENELM, wdtype=Q8, n_vocab=32000, n_embd=1536, n_layers=20,
                          n_heads=[12] * 3 + [16] * 7 + [20] * 6 + [24] * 4,
                          n_kv_heads=[3] * 3 + [4] * 7 + [5] * 6 + [6] * 4,
                          n_ffn=[768, 1024, 1280, 1536, 1792, 2304, 2560, 2816, 3072, 3328, 3584, 3840, 4096, 4352,
                                 4608, 5120, 5376, 5632, 5888, 6144],
                          eos=32002, rope_pct=1.0, prompt=64, gen=128, seed=0x5EED0007),
}
PROMPT_SEED_OFFSET = 0x1000


def workload_config(name, cls=ModelConfig, max_ctx=None):
    w = WORKLOADS[name]
    return make_config(w["arch"], w["wdtype"], w["n_vocab"], w["n_embd"], w["n_layers"], w["n_heads"],
                       w["n_kv_heads"], w["n_ffn"], max_ctx or (w["prompt"] + w["gen"]), eos=w["eos"],
                       rope_pct=w["rope_pct"], cls=cls)


def act_row_bytes_ref(dtype, cols):
    """Bytes of one activation row in the reference's layout."""
    if dtype == Q8:
        return (cols + 31) // 32 * 34
    return cols * (2 if dtype == F16 else 4)


def weight_bytes_ref(dtype, rows, cols):
    if dtype == Q8:
        return rows * (cols // 32) * 34
    if dtype == Q4:
        return rows * (cols // 32) * 18
    return rows * cols * 2


_lib = None

# nc_text_sink: void (*)(const char* text, void* user)
TEXT_SINK = C.CFUNCTYPE(None, C.c_char_p, C.c_void_p)


def lib():
    """The loaded product library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HipError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
    L = C.CDLL(LIB_PATH)
    VP, I, F, SZ, U64 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_uint64
    TP = C.POINTER(Tensor)
    sig = {
        "nc_init": (I, [I]), "nc_last_error": (C.c_char_p, []), "nc_malloc": (I, [C.POINTER(VP), SZ]),
        "nc_free": (I, [VP]), "nc_memcpy_h2d": (I, [VP, VP, SZ]), "nc_memcpy_d2h": (I, [VP, VP, SZ]),
        "nc_memset_d": (I, [VP, I, SZ]), "nc_synchronize": (I, []),
        "nc_act_pitch": (I, [I, I]), "nc_act_from_reference": (I, [VP, VP, I, I, I]),
        "nc_act_to_reference": (I, [VP, VP, I, I, I]),
        "nc_weight_bytes": (I, [I, I, I, C.POINTER(SZ), C.POINTER(SZ)]),
        "nc_weight_from_reference": (I, [VP, I, I, I, VP, VP]),
        "nc_gen_normal": (I, [U64, C.c_uint32, F, C.c_int64, VP, VP]),
        "nc_weight_quantize": (I, [VP, TP, VP]),
        "nc_token_embed": (I, [TP, VP, TP, I, I, VP]), "nc_matmul_2d": (I, [TP, TP, TP, I, I, VP]),
        "nc_rms_norm": (I, [TP, VP, TP, I, I, I, VP]), "nc_layer_norm": (I, [TP, VP, VP, TP, I, I, VP]),
        "nc_rotary_emb": (I, [TP, TP, I, F, VP, I, I, VP]), "nc_rope_table": (I, [I, I, F, VP]),
        "nc_silu": (I, [TP, TP, I, I, VP]), "nc_multiply": (I, [TP, TP, TP, I, I, VP]),
        "nc_add": (I, [TP, TP, TP, I, I, VP]), "nc_scale": (I, [TP, F, I, I, VP]),
        "nc_bias_add": (I, [TP, VP, I, I, VP]), "nc_qkv_attn": (I, [TP, TP, TP, TP, I, I, I, I, I, VP]),
        "nc_argmax": (I, [VP, I, VP, VP]), "nc_expf": (I, [VP, VP, C.c_int64, VP]),
        "nc_expf_host": (F, [F]), "nc_debug_spec": (I, [F, VP]),
        "nc_block_seq_sum_grid": (I, [VP, I, I, VP, VP, VP]),
        "nc_seq_sum_grid_host": (F, [VP, I, I, C.POINTER(I)]),
        "nc_model_create": (I, [C.POINTER(ModelConfig), C.POINTER(VP)]), "nc_model_free": (I, [VP]),
        "nc_model_init_synthetic": (I, [VP, U64]), "nc_model_set_weight": (I, [VP, I, I, VP, SZ]),
        "nc_model_get_weight": (I, [VP, I, I, VP, SZ]), "nc_model_logits": (I, [VP, VP, I, I, VP]),
        "nc_model_load_gten": (I, [VP, C.c_char_p]),
        "nc_model_generate_topk": (I, [VP, VP, I, I, C.c_float, I, C.c_uint32, VP, C.POINTER(I)]),
        "nc_rng_seed": (I, [C.c_uint32, VP]),
        "nc_sample_topk": (I, [VP, I, C.c_float, I, VP, VP, VP, VP]),
        "nc_exp": (I, [VP, VP, C.c_int64, VP]),
        "nc_exp_host": (C.c_double, [C.c_double]),
        "nc_tokenizer_load_bpe": (I, [C.c_char_p, I, I, C.c_char_p, C.c_char_p, VP, I, VP, I, C.POINTER(VP)]),
        "nc_tokenizer_load_words": (I, [C.c_char_p, I, I, VP, I, VP, I, C.POINTER(VP)]),
        "nc_tokenizer_load_for_model": (I, [C.c_char_p, C.c_char_p, C.POINTER(VP)]),
        "nc_tokenizer_encode": (I, [VP, C.c_char_p, VP, I, C.POINTER(I)]),
        "nc_tokenizer_decode": (C.c_char_p, [VP, I, I]),
        "nc_tokenizer_eos": (I, [VP]),
        "nc_tokenizer_free": (I, [VP]),
        "nc_model_layer_out": (I, [VP, I, I, VP]), "nc_model_generate": (I, [VP, VP, I, I, VP, C.POINTER(I)]),
        "nc_model_prefill": (I, [VP, VP, I]), "nc_model_decode": (I, [VP, I, VP]),
        "nc_model_profile_begin": (I, [VP, I]),
        "nc_model_profile_end": (I, [VP, C.POINTER(I)] + [C.POINTER(C.c_double)] * 4),
        "nc_model_profile_launches": (I, [VP, I, VP, VP, VP, C.POINTER(I)]),
        "nc_copy_d2d": (I, [VP, VP, C.c_size_t, VP]),
        "nc_model_sample_begin": (I, [VP, VP, I, F, I, C.c_uint32]),
        "nc_model_sample_steps": (I, [VP, I, VP]),
        "nc_model_get_config": (I, [VP, C.POINTER(ModelConfig)]),
        "nc_greedy_sample": (I, [VP, VP, C.c_char_p, I, TEXT_SINK, VP, C.POINTER(I)]),
        "nc_topk_sample": (I, [VP, VP, C.c_char_p, I, F, I, C.c_uint32, TEXT_SINK, VP, C.POINTER(I)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    _lib = L
    return L


def check(status, what=""):
    if status != 0:
        msg = lib().nc_last_error().decode(errors="replace")
        raise HipError(f"{what}: status {status}: {msg}")


def init(device=0):
    check(lib().nc_init(device), "nc_init")


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


# Launch roles of nc_model_profile_launches (NC_PROF_* in gten_hip.h).
PROF_ROLES = {0: "qkv", 1: "o", 2: "gate_up", 3: "down", 4: "lm_head"}
PROF_FUSED = 8


class Tokenizer:
    """The reference's tokenizers (gten/tokenizer.cpp) on the host.

    Tokenizer.for_model("tinyllama", path) builds the one nanochat.cpp uses
    for that model; bpe(...) / words(...) take the constructor arguments of
    LLamaTokenizer / Gpt2Tokenizer.  encode(str) -> int32 array,
    decode(prev, token) -> bytes (a piece may be part of a UTF-8 character).
    """

    def __init__(self, handle):
        self.h = handle

    @classmethod
    def for_model(cls, model, path):
        h = C.c_void_p()
        check(lib().nc_tokenizer_load_for_model(model.encode(), os.fsencode(path), C.byref(h)), "tokenizer")
        return cls(h)

    @classmethod
    def bpe(cls, path, vocab_size, eos, prompt_prefix="", prompt_suffix="", tokens_prefix=(), tokens_suffix=()):
        import numpy as np
        pre = np.ascontiguousarray(tokens_prefix, np.int32)
        suf = np.ascontiguousarray(tokens_suffix, np.int32)
        h = C.c_void_p()
        check(lib().nc_tokenizer_load_bpe(os.fsencode(path), vocab_size, eos, prompt_prefix.encode(),
                                          prompt_suffix.encode(), _ptr(pre), len(pre), _ptr(suf), len(suf),
                                          C.byref(h)), "tokenizer")
        return cls(h)

    @classmethod
    def words(cls, path, vocab_size, eos, tokens_prefix=(), tokens_suffix=()):
        import numpy as np
        pre = np.ascontiguousarray(tokens_prefix, np.int32)
        suf = np.ascontiguousarray(tokens_suffix, np.int32)
        h = C.c_void_p()
        check(lib().nc_tokenizer_load_words(os.fsencode(path), vocab_size, eos, _ptr(pre), len(pre), _ptr(suf),
                                            len(suf), C.byref(h)), "tokenizer")
        return cls(h)

    def encode(self, text):
        import numpy as np
        b = text.encode() if isinstance(text, str) else bytes(text)
        n = C.c_int()
        cap = 2 * len(b) + 64
        out = np.zeros(cap, np.int32)
        st = lib().nc_tokenizer_encode(self.h, b, _ptr(out), cap, C.byref(n))
        if st != 0 and n.value > cap:  # room for the count the first call reported
            out = np.zeros(n.value, np.int32)
            st = lib().nc_tokenizer_encode(self.h, b, _ptr(out), n.value, C.byref(n))
        check(st, "encode")
        return out[: n.value]

    def decode(self, prev_token, token):
        return lib().nc_tokenizer_decode(self.h, prev_token, token) or b""

    @property
    def eos(self):
        return lib().nc_tokenizer_eos(self.h)

    def close(self):
        if self.h:
            lib().nc_tokenizer_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceBuffer:
    """An HBM allocation owned by Python (freed on close/GC)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().nc_malloc(C.byref(p), max(self.nbytes, 16)), "nc_malloc")
        self.ptr = p.value

    def upload(self, arr, offset=0):
        check(lib().nc_memcpy_h2d(C.c_void_p(self.ptr + offset), _ptr(arr), arr.nbytes), "h2d")

    def download(self, arr, offset=0):
        check(lib().nc_memcpy_d2h(_ptr(arr), C.c_void_p(self.ptr + offset), arr.nbytes), "d2h")
        return arr

    def close(self):
        if self.ptr:
            lib().nc_free(C.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    """gten::Model on the device (nc_model_*)."""

    def __init__(self, cfg):
        self.cfg = cfg
        h = C.c_void_p()
        check(lib().nc_model_create(C.byref(cfg), C.byref(h)), "nc_model_create")
        self.h = h

    def init_synthetic(self, seed):
        check(lib().nc_model_init_synthetic(self.h, seed), "init_synthetic")

    def load_gten(self, path):
        """Model::load_from_ckpt: every weight from a .gten checkpoint file."""
        check(lib().nc_model_load_gten(self.h, os.fsencode(path)), "load_gten")

    def set_weight(self, layer, slot, ref_bytes):
        check(lib().nc_model_set_weight(self.h, layer, slot, _ptr(ref_bytes), ref_bytes.nbytes), "set_weight")

    def get_weight(self, layer, slot, nbytes):
        import numpy as np
        out = np.zeros(nbytes, np.uint8)
        check(lib().nc_model_get_weight(self.h, layer, slot, _ptr(out), nbytes), "get_weight")
        return out

    def logits(self, tokens, start_pos):
        import numpy as np
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros(self.cfg.n_vocab, np.float32)
        check(lib().nc_model_logits(self.h, _ptr(toks), len(toks), start_pos, _ptr(out)), "logits")
        return out

    def layer_out(self, layer, row):
        import numpy as np
        adt = F16 if self.cfg.wdtype == F16 else Q8
        out = np.zeros(act_row_bytes_ref(adt, self.cfg.n_embd), np.uint8)
        check(lib().nc_model_layer_out(self.h, layer, row, _ptr(out)), "layer_out")
        return out

    def generate(self, prompt, n_gen):
        import numpy as np
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_gen, np.int32)
        n = C.c_int()
        check(lib().nc_model_generate(self.h, _ptr(p), len(p), n_gen, _ptr(out), C.byref(n)), "generate")
        return out[: n.value]

    def generate_topk(self, prompt, n_gen, temp, top_k, seed):
        """topk_sample with std::mt19937(seed): up to n_gen sampled tokens."""
        import numpy as np
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_gen, np.int32)
        n = C.c_int()
        check(lib().nc_model_generate_topk(self.h, _ptr(p), len(p), n_gen, temp, top_k, seed, _ptr(out), C.byref(n)),
              "generate_topk")
        return out[: n.value]

    def prefill(self, prompt):
        import numpy as np
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        check(lib().nc_model_prefill(self.h, _ptr(p), len(p)), "prefill")

    def decode(self, n_steps, fetch=False):
        """n_steps more greedy steps; with fetch, returns every token
        generated since the prompt (the first one included)."""
        if not fetch:
            check(lib().nc_model_decode(self.h, n_steps, None), "decode")
            return None
        import numpy as np
        out = np.zeros(self.cfg.max_ctx + 1, np.int32)
        check(lib().nc_model_decode(self.h, n_steps, _ptr(out)), "decode")
        return out

    def profile_begin(self, max_launches):
        check(lib().nc_model_profile_begin(self.h, max_launches), "profile_begin")

    def profile_end(self):
        n = C.c_int()
        vals = [C.c_double() for _ in range(4)]
        check(lib().nc_model_profile_end(self.h, C.byref(n), *[C.byref(v) for v in vals]), "profile_end")
        total_ms, total_bytes, min_ms, max_ms = (v.value for v in vals)
        return dict(launches=n.value, total_ms=total_ms, total_bytes=total_bytes, min_ms=min_ms, max_ms=max_ms)

    def profile_launches(self, cap):
        """Per-launch (ms, algorithmic bytes, role) of the profiled launches."""
        import numpy as np
        ms = np.zeros(cap, np.float32)
        by = np.zeros(cap, np.float64)
        kind = np.zeros(cap, np.int32)
        n = C.c_int()
        check(lib().nc_model_profile_launches(self.h, cap, _ptr(ms), _ptr(by), _ptr(kind), C.byref(n)),
              "profile_launches")
        return ms[: n.value], by[: n.value], kind[: n.value]

    def close(self):
        if self.h:
            lib().nc_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _sample_text(call, on_text):
    pieces = []

    def sink(text, _user):
        piece = text or b""
        pieces.append(piece)
        if on_text:
            on_text(piece)

    cb = TEXT_SINK(sink)
    n = C.c_int()
    check(call(cb, C.byref(n)), "sample")
    return b"".join(pieces), n.value


def greedy_sample(model, tokenizer, prompt, n_predict=0, on_text=None):
    """greedy_sample (src/gten/sampler.cpp:11-60) end to end: prompt text
    (str or bytes) in, the text the reference writes out (bytes, closing
    newline included) and the number of tokens generated.  on_text(piece)
    sees each decoded piece as it is produced.  n_predict <= 0: the model's
    max_ctx."""
    p = prompt.encode() if isinstance(prompt, str) else bytes(prompt)
    return _sample_text(lambda cb, n: lib().nc_greedy_sample(model.h, tokenizer.h, p, n_predict, cb, None, n),
                        on_text)


def topk_sample(model, tokenizer, prompt, temp=0.9, top_k=50, seed=0, n_predict=0, on_text=None):
    """topk_sample (src/gten/sampler.cpp:63-143) end to end, with
    std::mt19937(seed) in place of the random_device seed."""
    p = prompt.encode() if isinstance(prompt, str) else bytes(prompt)
    return _sample_text(
        lambda cb, n: lib().nc_topk_sample(model.h, tokenizer.h, p, n_predict, temp, top_k, seed, cb, None, n),
        on_text)
