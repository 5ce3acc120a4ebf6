"""Op-level parity of the HIP kernels with the oracle, through the C-ABI.

Every op of gten::ops (src/gten/ops.h:10-40) runs on the device and in the
oracle on the same seeded inputs (reference byte layouts); results must be
byte-identical: activation rows (Q8 codes + fp16 deltas, fp16 values) and
raw fp32 dot products alike.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as OL
from devutil import DevAct, DevWeight, dev_array, ptr, sync

pytestmark = pytest.mark.gpu

Q8, Q4, F16, F32 = OL.Q8, OL.Q4, OL.F16, OL.F32


def rand_act(oracle, rng, dtype, rows, cols, scale=1.0):
    x = (rng.standard_normal((rows, cols)) * scale).astype(np.float32)
    if dtype == F32:
        return x
    if dtype == F16:
        return x.astype(np.float16).view(np.uint16)
    out = np.zeros((rows, OL.row_bytes(Q8, cols)), np.uint8)
    for r in range(rows):
        oracle.q8_quantize_row(OL.ptr(x[r]), OL.ptr(out[r]), cols)
    return out


def rand_weight(oracle, rng, dtype, rows, cols, scale=0.02):
    w = (rng.standard_normal((rows, cols)) * scale).astype(np.float32)
    if dtype == F16:
        return w.astype(np.float16).view(np.uint16)
    out = np.zeros((rows, OL.row_bytes(dtype, cols)), np.uint8)
    fn = oracle.q8_quantize_weights if dtype == Q8 else oracle.q4_quantize_weights
    fn(OL.ptr(w), rows * cols // 32, OL.ptr(out))
    return out


def assert_same(got, want, what):
    got = np.ascontiguousarray(got).view(np.uint8).reshape(-1)
    want = np.ascontiguousarray(want).view(np.uint8).reshape(-1)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{what}: {bad.size} of {got.size} bytes differ, first at {bad[:8]}"


MATMUL_CASES = [
    # (x dtype, w dtype, K, N, rows, start)
    (Q8, Q4, 2048, 2048, 1, 0),
    (Q8, Q4, 5632, 2048, 1, 0),
    (Q8, Q4, 2048, 11264, 1, 0),
    (Q8, Q4, 2304, 250, 3, 1),
    (Q8, Q8, 2048, 2560, 1, 0),
    (Q8, Q8, 8192, 2048, 1, 0),
    (Q8, Q8, 64, 40, 5, 2),
    (Q8, Q4, 1024, 96, 9, 0),
    # prompt-row shapes: every launch shape of the prefill matmul's table
    # (fp16 matrix cores: 8- and 4-block chunks, short / medium / long
    # prompts, tall weights, columns past a 16-multiple; the integer kernel
    # for long prompts of tall weights and for rows of K % 128 != 0)
    (Q8, Q4, 2048, 2560, 64, 0),
    (Q8, Q4, 2048, 2048, 40, 3),
    (Q8, Q4, 5632, 2048, 16, 0),
    (Q8, Q8, 2048, 9000, 24, 0),
    (Q8, Q8, 2304, 300, 100, 7),
    (Q8, Q4, 5760, 1000, 50, 0),
    (Q8, Q4, 1152, 3000, 60, 0),
    (Q8, Q4, 2048, 8192, 260, 0),
    (Q8, Q4, 2048, 700, 300, 0),
    (Q8, Q8, 192, 100, 12, 0),
    (F16, F16, 2048, 2048, 1, 0),
    (F16, F16, 5632, 2048, 1, 0),
    (F16, F16, 128, 44, 4, 1),
    (F16, F16, 2304, 250, 1, 0),
    (F16, F16, 5760, 2304, 1, 0),
    (F16, F16, 2048, 100, 1, 0),
    (F16, F16, 1280, 96, 1, 0),
    (F16, F16, 2048, 2048, 64, 0),
    (F16, F16, 5632, 2048, 16, 3),
    (F16, F16, 2048, 300, 13, 0),
    (F16, F16, 256, 768, 9, 1),
]


@pytest.mark.parametrize("xdt,wdt,K,N,rows,start", MATMUL_CASES)
def test_matmul_fp32_out(gpu, oracle, xdt, wdt, K, N, rows, start):
    rng = np.random.default_rng(K * 7 + N)
    x = rand_act(oracle, rng, xdt, rows, K)
    w = rand_weight(oracle, rng, wdt, N, K)
    want = np.zeros((rows, N), np.float32)
    oracle.matmul(OL.ptr(x), xdt, OL.ptr(w), wdt, OL.ptr(want), F32, K, N, start, rows, None)
    dx, dw = DevAct(x, xdt, rows, K), DevWeight(w, wdt, N, K)
    out = DevAct.empty(F32, rows, N)
    gpu.check(gpu.lib().nc_matmul_2d(C.byref(dx.t), C.byref(dw.t), C.byref(out.t), start, rows, None), "matmul")
    got = out.ref().view(np.float32)
    assert_same(got[start:], want[start:], f"matmul {xdt}x{wdt} K={K} N={N}")


@pytest.mark.parametrize("xdt,wdt,K,N", [(Q8, Q4, 2048, 256), (Q8, Q8, 2048, 512), (F16, F16, 2048, 320)])
def test_matmul_act_out(gpu, oracle, xdt, wdt, K, N):
    rng = np.random.default_rng(N)
    rows = 3
    x = rand_act(oracle, rng, xdt, rows, K)
    w = rand_weight(oracle, rng, wdt, N, K)
    want = np.zeros((rows, OL.row_bytes(xdt, N)), np.uint8)
    oracle.matmul(OL.ptr(x), xdt, OL.ptr(w), wdt, OL.ptr(want), xdt, K, N, 0, rows, None)
    dx, dw, out = DevAct(x, xdt, rows, K), DevWeight(w, wdt, N, K), DevAct.empty(xdt, rows, N)
    gpu.check(gpu.lib().nc_matmul_2d(C.byref(dx.t), C.byref(dw.t), C.byref(out.t), 0, rows, None), "matmul")
    assert_same(out.ref(), want, "matmul act out")


@pytest.mark.parametrize("dt", [Q8, F16])
@pytest.mark.parametrize("d,scale", [(2048, 1.0), (2304, 30.0), (256, 0.01)])
def test_rms_norm(gpu, oracle, dt, d, scale):
    rng = np.random.default_rng(d)
    rows, start = 4, 1
    x = rand_act(oracle, rng, dt, rows, d, scale)
    w = (1 + 0.2 * rng.standard_normal(d)).astype(np.float16).view(np.uint16)
    want = np.zeros_like(x)
    oracle.rms_norm(OL.ptr(x), dt, OL.ptr(w), OL.ptr(want), d, start, rows)
    dx, out, dwt = DevAct(x, dt, rows, d), DevAct.empty(dt, rows, d), dev_array(w)
    gpu.check(gpu.lib().nc_rms_norm(C.byref(dx.t), C.c_void_p(dwt.ptr), C.byref(out.t), d, start, rows, None), "rms")
    assert_same(out.ref()[start:], want[start:], "rms_norm")


@pytest.mark.parametrize("dt", [Q8, F16])
def test_rms_norm_per_head(gpu, oracle, dt):
    rng = np.random.default_rng(5)
    rows, heads = 3, 20
    d = heads * 64
    x = rand_act(oracle, rng, dt, rows, d)
    w = (1 + 0.2 * rng.standard_normal(64)).astype(np.float16).view(np.uint16)
    want = np.zeros_like(x)
    oracle.rms_norm_heads(OL.ptr(x), dt, OL.ptr(w), OL.ptr(want), heads, 64, 0, rows)
    dx, out, dwt = DevAct(x, dt, rows, d), DevAct.empty(dt, rows, d), dev_array(w)
    gpu.check(gpu.lib().nc_rms_norm(C.byref(dx.t), C.c_void_p(dwt.ptr), C.byref(out.t), 64, 0, rows, None), "rms3d")
    assert_same(out.ref(), want, "rms_norm per head")


@pytest.mark.parametrize("dt", [Q8, F16])
def test_layer_norm(gpu, oracle, dt):
    rng = np.random.default_rng(11)
    rows, d = 3, 2048
    x = rand_act(oracle, rng, dt, rows, d, 2.0)
    x_f = rng.standard_normal(d)
    w = (1 + 0.2 * x_f).astype(np.float16).view(np.uint16)
    b = (0.1 * rng.standard_normal(d)).astype(np.float16).view(np.uint16)
    want = np.zeros_like(x)
    oracle.layer_norm(OL.ptr(x), dt, OL.ptr(w), OL.ptr(b), OL.ptr(want), d, 0, rows)
    dx, out, dw_, db_ = DevAct(x, dt, rows, d), DevAct.empty(dt, rows, d), dev_array(w), dev_array(b)
    gpu.check(gpu.lib().nc_layer_norm(C.byref(dx.t), C.c_void_p(dw_.ptr), C.c_void_p(db_.ptr), C.byref(out.t), 0,
                                      rows, None), "layer_norm")
    assert_same(out.ref(), want, "layer_norm")


@pytest.mark.parametrize("dt", [Q8, F16])
@pytest.mark.parametrize("pct,start", [(1.0, 0), (0.25, 5), (1.0, 300)])
def test_rotary_emb(gpu, oracle, dt, pct, start):
    rng = np.random.default_rng(int(pct * 100) + start)
    rows, d = start + 4, 2048
    x = rand_act(oracle, rng, dt, rows, d, 3.0)
    want = x.copy()
    oracle.rotary_emb(OL.ptr(x), OL.ptr(want), dt, d, 64, pct, start, rows)
    d_half = int(64 * pct) // 2
    tab = np.zeros((rows, max(d_half, 1), 2), np.float32)
    gpu.check(gpu.lib().nc_rope_table(rows, 64, pct, ptr(tab)), "rope_table")
    dtab = dev_array(tab)
    dx = DevAct(x, dt, rows, d)
    out = DevAct(x, dt, rows, d)
    gpu.check(gpu.lib().nc_rotary_emb(C.byref(dx.t), C.byref(out.t), 64, pct, C.c_void_p(dtab.ptr), start, rows, None),
              "rope")
    assert_same(out.ref()[start:], want[start:], "rotary_emb")


SCALE = float(np.float32(1.4 / 40 ** 0.5))


@pytest.mark.parametrize("dt", [Q8, F16])
@pytest.mark.parametrize("op", ["silu", "mul", "add", "scale", "bias"])
def test_elementwise(gpu, oracle, dt, op):
    rng = np.random.default_rng(["silu", "mul", "add", "scale", "bias"].index(op))
    rows, d = 3, 5632
    a = rand_act(oracle, rng, dt, rows, d, 4.0)
    b = rand_act(oracle, rng, dt, rows, d, 1.0)
    bias = (0.3 * rng.standard_normal(d)).astype(np.float16).view(np.uint16)
    want = a.copy()
    if op == "silu":
        oracle.silu(OL.ptr(a), OL.ptr(want), dt, d, 0, rows)
    elif op == "mul":
        oracle.multiply(OL.ptr(a), OL.ptr(b), OL.ptr(want), dt, d, 0, rows)
    elif op == "add":
        oracle.add(OL.ptr(a), OL.ptr(b), OL.ptr(want), dt, d, 0, rows)
    elif op == "scale":
        oracle.scale(OL.ptr(want), dt, SCALE, d, 0, rows)
    else:
        oracle.bias_add(OL.ptr(want), dt, OL.ptr(bias), d, 0, rows)
    da, db_, out, dbias = DevAct(a, dt, rows, d), DevAct(b, dt, rows, d), DevAct.empty(dt, rows, d), dev_array(bias)
    L = gpu.lib()
    if op == "silu":
        st = L.nc_silu(C.byref(da.t), C.byref(out.t), 0, rows, None)
    elif op == "mul":
        st = L.nc_multiply(C.byref(da.t), C.byref(db_.t), C.byref(out.t), 0, rows, None)
    elif op == "add":
        st = L.nc_add(C.byref(da.t), C.byref(db_.t), C.byref(out.t), 0, rows, None)
    elif op == "scale":
        st = L.nc_scale(C.byref(da.t), SCALE, 0, rows, None)
        out = da
    else:
        st = L.nc_bias_add(C.byref(da.t), C.c_void_p(dbias.ptr), 0, rows, None)
        out = da
    gpu.check(st, op)
    assert_same(out.ref(), want, op)


ATTN_CASES = [
    # (dtype, n_heads, n_kv_heads, n_ctx, start)
    (Q8, 32, 4, 320, 319),
    (Q8, 32, 4, 1, 0),
    (Q8, 36, 36, 640, 639),
    (Q8, 20, 5, 77, 76),
    (Q8, 8, 2, 64, 0),
    (Q8, 4, 1, 100, 37),
    (F16, 32, 32, 256, 255),
    (F16, 4, 4, 128, 0),
    (F16, 8, 2, 45, 20),
    # contexts of the reference's models: 1024 (its default), 2048, 4096; the
    # single-row softmax sum changes from one wavefront's loop to the exact
    # workgroup sum above 1024 positions; n mod 8 / mod 32 edges; the prefill
    # kernel's 8, 4 and 2 rows per workgroup (m <= 1024, <= 2048, beyond)
    (Q8, 32, 4, 1024, 1023),
    (Q8, 32, 4, 1025, 1024),
    (Q8, 32, 4, 1031, 1030),
    (Q8, 36, 36, 2048, 2047),
    (Q8, 16, 4, 2053, 2040),
    (Q8, 32, 4, 4096, 4095),
    (Q8, 4, 1, 4093, 4080),
    (Q8, 8, 2, 1100, 0),
    (Q8, 4, 1, 3000, 0),
    (F16, 32, 32, 1024, 1023),
    (F16, 32, 32, 2049, 2048),
    (F16, 32, 32, 4096, 4095),
    (F16, 4, 4, 4090, 4081),
    (F16, 4, 2, 1500, 0),
]


@pytest.mark.parametrize("dt,hq,hkv,n,start", ATTN_CASES)
def test_qkv_attn(gpu, oracle, dt, hq, hkv, n, start):
    rng = np.random.default_rng(hq * 1000 + n)
    q = rand_act(oracle, rng, dt, n, hq * 64, 2.0)
    k = rand_act(oracle, rng, dt, n, hkv * 64, 2.0)
    v = rand_act(oracle, rng, dt, n, hkv * 64, 1.0)
    want = np.zeros((n, OL.row_bytes(dt, hq * 64)), np.uint8)
    oracle.qkv_attn(OL.ptr(q), OL.ptr(k), OL.ptr(v), OL.ptr(want), dt, hq, hkv, 64, start, n)
    dq, dk, dv = DevAct(q, dt, n, hq * 64), DevAct(k, dt, n, hkv * 64), DevAct(v, dt, n, hkv * 64)
    out = DevAct.empty(dt, n, hq * 64)
    gpu.check(gpu.lib().nc_qkv_attn(C.byref(dq.t), C.byref(dk.t), C.byref(dv.t), C.byref(out.t), hq, hkv, 64, start,
                                    n, None), "qkv_attn")
    assert_same(out.ref()[start:], want[start:], "qkv_attn")


@pytest.mark.parametrize("wdt", [Q4, Q8, F16])
def test_token_embed(gpu, oracle, wdt):
    rng = np.random.default_rng(wdt)
    vocab, d, rows = 1000, 2048, 6
    table = rand_weight(oracle, rng, wdt, vocab, d, 0.5)
    adt = F16 if wdt == F16 else Q8
    toks = np.array([0, 999, 5, 5, 123, 640], np.int32)
    want = np.zeros((rows, OL.row_bytes(adt, d)), np.uint8)
    oracle.token_embed(OL.ptr(table), wdt, OL.ptr(toks), OL.ptr(want), adt, d, vocab, 0, rows)
    dtab, dtok, out = DevWeight(table, wdt, vocab, d), dev_array(toks), DevAct.empty(adt, rows, d)
    gpu.check(gpu.lib().nc_token_embed(C.byref(dtab.t), C.c_void_p(dtok.ptr), C.byref(out.t), 0, rows, None), "embed")
    assert_same(out.ref(), want, "token_embed")


@pytest.mark.parametrize("n", [1, 1000, 32000, 122753])
def test_argmax_first_max(gpu, oracle, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    if n > 10:
        x[n // 3] = x[n // 2] = x[n - 1] = 9.0  # ties: the first index wins
    dx = dev_array(x)
    out = np.zeros(1, np.int32)
    dout = dev_array(out)
    gpu.check(gpu.lib().nc_argmax(C.c_void_p(dx.ptr), n, C.c_void_p(dout.ptr), None), "argmax")
    dout.download(out)
    assert out[0] == oracle.argmax(OL.ptr(x), n)


def test_weight_generation_and_quantization(gpu, oracle):
    """Device generator + quantizer equal the oracle's bit for bit."""
    L = gpu.lib()
    n = 2048 * 512
    want_f = np.zeros(n, np.float32)
    oracle.gen_normal(77, 13, 0.02, n, OL.ptr(want_f))
    dbuf = gpu.DeviceBuffer(n * 4)
    gpu.check(L.nc_gen_normal(77, 13, 0.02, n, C.c_void_p(dbuf.ptr), None), "gen_normal")
    got_f = np.zeros(n, np.float32)
    sync()
    dbuf.download(got_f)
    assert_same(got_f, want_f, "gen_normal")
    for dt in (Q8, Q4, F16):
        rows, cols = 512, 2048
        want = np.zeros(rows * OL.row_bytes(dt, cols), np.uint8)
        if dt == F16:
            want = want_f.astype(np.float16).view(np.uint8)
        else:
            (oracle.q8_quantize_weights if dt == Q8 else oracle.q4_quantize_weights)(OL.ptr(want_f), n // 32,
                                                                                    OL.ptr(want))
        w = DevWeight(np.zeros_like(want), dt, rows, cols)
        gpu.check(L.nc_weight_quantize(C.c_void_p(dbuf.ptr), C.byref(w.t), None), "weight_quantize")
        sync()
        cb = np.zeros(w.cbuf.nbytes, np.uint8)
        w.cbuf.download(cb)
        want_codes = np.zeros_like(cb)
        want_deltas = np.zeros(w.dbuf.nbytes, np.uint8)
        gpu.check(L.nc_weight_from_reference(ptr(want), dt, rows, cols, ptr(want_codes), ptr(want_deltas)), "repack")
        assert_same(cb, want_codes, f"codes dtype {dt}")
        if dt != F16:
            db_ = np.zeros(w.dbuf.nbytes, np.uint8)
            w.dbuf.download(db_)
            assert_same(db_, want_deltas, f"deltas dtype {dt}")


def test_expf_exhaustive(gpu, oracle):
    """Device std::exp(float) equals the host glibc expf on all 2^32 inputs."""
    L = gpu.lib()
    chunk = 1 << 27
    dx, dy = gpu.DeviceBuffer(chunk * 4), gpu.DeviceBuffer(chunk * 4)
    y = np.zeros(chunk, np.float32)
    f = oracle.lib.or_expf_mismatches
    f.restype, f.argtypes = C.c_int64, [C.c_void_p, C.c_void_p, C.c_int64, C.POINTER(C.c_int64)]
    total = 0
    first = []
    for start in range(0, 1 << 32, chunk):
        x = np.arange(start, start + chunk, dtype=np.uint64).astype(np.uint32).view(np.float32)
        dx.upload(x)
        gpu.check(L.nc_expf(C.c_void_p(dx.ptr), C.c_void_p(dy.ptr), chunk, None), "expf")
        sync()
        dy.download(y)
        fi = C.c_int64()
        cnt = f(OL.ptr(x), OL.ptr(y), chunk, C.byref(fi))
        total += cnt
        if cnt and len(first) < 8:
            first.append((hex(int(x.view(np.uint32)[fi.value])), float(y[fi.value])))
    assert total == 0, f"{total} inputs differ from glibc expf, e.g. {first}"
