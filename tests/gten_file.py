"""Writing and reading .gten checkpoints in the converters' layout
(tinyllama/tinyllama_to_gten.py:94-201, zephyr1_6b_to_gten.py, minicpm_to_gten.py,
openelm_to_gten.py): an 8-byte magic number, then per tensor a layer header
(int32 name size, name) and a weight record (int32 name size, name, int32
payload size, payload), the payload being Q8 / Q4 blocks (fp16 delta, then 32
codes / 16 packed bytes) or fp16 values.  The tensor order is each model's
load_from_ckpt order (tinyllama/tinyllama.cpp:131-187, zephyr/zephyr.cpp:79-150,
minicpm/minicpm.cpp:113-166, openelm/openelm.cpp:201-262).

Test infrastructure: files are written from the oracle's synthetic weights."""
import struct

import numpy as np

import oracle_lib as OL

MAGIC = 0x454C49464E455447

# weight slots (the product's and the oracle's numbering)
W_Q, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN = range(7)
W_ATTN_NORM, W_ATTN_NORM_B, W_MLP_NORM, W_MLP_NORM_B = 7, 8, 9, 10
W_Q_BIAS, W_K_BIAS, W_V_BIAS, W_Q_NORM, W_K_NORM = 11, 12, 13, 14, 15
TID_EMB, TID_NORM, TID_NORM_B, TID_LM = 0xFFFF0, 0xFFFF1, 0xFFFF2, 0xFFFF3
LLAMA, ZEPHYR, MINICPM, OPENELM = 0, 1, 2, 3

_NAMES = {W_Q: "self_attn.q_proj.weight", W_K: "self_attn.k_proj.weight", W_V: "self_attn.v_proj.weight",
          W_O: "self_attn.o_proj.weight", W_GATE: "mlp.gate_proj.weight", W_UP: "mlp.up_proj.weight",
          W_DOWN: "mlp.down_proj.weight", W_ATTN_NORM: "input_layernorm.weight",
          W_ATTN_NORM_B: "input_layernorm.bias", W_MLP_NORM: "post_attention_layernorm.weight",
          W_MLP_NORM_B: "post_attention_layernorm.bias", W_Q_BIAS: "self_attn.q_proj.bias",
          W_K_BIAS: "self_attn.k_proj.bias", W_V_BIAS: "self_attn.v_proj.bias",
          W_Q_NORM: "attn.q_norm.weight", W_K_NORM: "attn.k_norm.weight"}


def order(cfg):
    """(layer, slot, name) of every tensor of a model, in file order."""
    out = [(-1, TID_EMB, "model.embed_tokens.weight")]
    for l in range(cfg.n_layers):
        if cfg.arch == ZEPHYR:
            slots = [W_Q, W_Q_BIAS, W_K, W_K_BIAS, W_V, W_V_BIAS, W_O, W_GATE, W_UP, W_DOWN,
                     W_ATTN_NORM, W_ATTN_NORM_B, W_MLP_NORM, W_MLP_NORM_B]
        else:
            slots = [W_Q, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN]
            if cfg.arch == OPENELM:
                slots += [W_Q_NORM, W_K_NORM]
            slots += [W_ATTN_NORM, W_MLP_NORM]
        out += [(l, s, f"model.layers.{l}.{_NAMES[s]}") for s in slots]
    out.append((-1, TID_NORM, "model.norm.weight"))
    if cfg.arch == ZEPHYR:
        out.append((-1, TID_NORM_B, "model.norm.bias"))
    if cfg.arch in (LLAMA, ZEPHYR):
        out.append((-1, TID_LM, "lm_head.weight"))
    return out


def weight_bytes(oracle, cfg, seed, layer, slot):
    """The oracle's synthetic weight (layer, slot) in the reference's storage."""
    rows, cols, dt = oracle.weight_shape(cfg, layer, slot)
    buf = np.zeros(rows * OL.row_bytes(dt, cols), np.uint8)
    oracle.make_weight(OL.C.byref(cfg), seed, layer, slot, OL.ptr(buf))
    return buf


_VECTOR_SLOTS = (W_ATTN_NORM, W_ATTN_NORM_B, W_MLP_NORM, W_MLP_NORM_B, W_Q_BIAS, W_K_BIAS, W_V_BIAS,
                 W_Q_NORM, W_K_NORM, TID_NORM, TID_NORM_B)


def distinct_vectors(layer, slot, data):
    """payload_fn giving every fp16 norm gain / bias its own values (the
    synthetic gains are all 1 and the biases 0, so records in a wrong order
    would go unnoticed): gains 1 + N(0, 0.1), biases N(0, 0.05), drawn from a
    generator seeded by the tensor."""
    if slot not in _VECTOR_SLOTS:
        return data
    n = len(data) // 2
    rng = np.random.default_rng([layer + 1, slot])
    gain = slot in (W_ATTN_NORM, W_MLP_NORM, W_Q_NORM, W_K_NORM, TID_NORM)
    v = 1.0 + 0.1 * rng.standard_normal(n) if gain else 0.05 * rng.standard_normal(n)
    return v.astype(np.float16).tobytes()


def scaled_embedding(factor, q8):
    """payload_fn scaling the embedding's Q8 (q8) or Q4 block deltas (fp16,
    rounded to nearest) by factor; other tensors unchanged."""
    def fn(layer, slot, data):
        if slot != TID_EMB:
            return data
        return scale_block_deltas(np.frombuffer(data, np.uint8), q8, factor).tobytes()
    return fn


def scale_block_deltas(buf, q8, factor):
    """Q8 (34-byte) or Q4 (18-byte) blocks with every fp16 delta times factor."""
    blk = np.array(buf, np.uint8).reshape(-1, 34 if q8 else 18)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32) * np.float32(factor)
    blk[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return blk.reshape(-1)


def workload_weight(oracle, cfg, w, layer, slot):
    """Weight (layer, slot) of a workload dict: the synthetic one, with the
    embedding deltas scaled when the workload has emb_scale."""
    data = weight_bytes(oracle, cfg, w["seed"], layer, slot)
    if slot == TID_EMB and w.get("emb_scale"):
        data = scale_block_deltas(data, cfg.wdtype == OL.Q8, w["emb_scale"])
    return data


def payloads(cfg, seed, oracle, payload_fn=None):
    """{(layer, slot): payload bytes} of every tensor of the model."""
    out = {}
    for layer, slot, _ in order(cfg):
        data = weight_bytes(oracle, cfg, seed, layer, slot).tobytes()
        out[(layer, slot)] = payload_fn(layer, slot, data) if payload_fn is not None else data
    return out


def _name(b):
    return struct.pack("<i", len(b)) + b


def write(path, cfg, seed, oracle, payload_fn=None, magic=MAGIC, truncate=None):
    """Writes the synthetic model (cfg, seed) as a .gten file.  payload_fn
    (layer, slot, bytes) -> bytes may replace a payload; truncate cuts the
    file to that many bytes."""
    parts = [struct.pack("<q", magic)]
    for layer, slot, name in order(cfg):
        data = weight_bytes(oracle, cfg, seed, layer, slot).tobytes()
        if payload_fn is not None:
            data = payload_fn(layer, slot, data)
        nb = name.encode()
        parts += [_name(nb), _name(nb), struct.pack("<i", len(data)), data]
    blob = b"".join(parts)
    if truncate is not None:
        blob = blob[:truncate]
    with open(path, "wb") as f:
        f.write(blob)


def read(path):
    """(magic, [(layer name, weight name, payload bytes)]) of a .gten file."""
    with open(path, "rb") as f:
        blob = f.read()
    (magic,) = struct.unpack_from("<q", blob, 0)
    off, recs = 8, []
    while off < len(blob):
        names = []
        for _ in range(2):
            (n,) = struct.unpack_from("<i", blob, off)
            names.append(blob[off + 4:off + 4 + n].decode())
            off += 4 + n
        (size,) = struct.unpack_from("<i", blob, off)
        recs.append((names[0], names[1], blob[off + 4:off + 4 + size]))
        off += 4 + size
    return magic, recs
