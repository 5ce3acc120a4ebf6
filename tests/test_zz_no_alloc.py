"""nc_matmul_2d_noalloc (the allocation-free matmul_2d) against nc_matmul_2d.

Two calls in a row through the C-ABI, the second with a smaller input (the
staging array keeps the first call's contents), for Q8 and fp16 activation
outputs: every output byte must equal the allocating entry point's and the
oracle's.  A call whose staging would not fit the array is refused.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as OL
from devutil import DevAct, DevWeight, sync

pytestmark = pytest.mark.gpu

Q8, Q4, F16 = OL.Q8, OL.Q4, OL.F16


def rand_act(oracle, rng, dtype, rows, cols):
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    if dtype == F16:
        return x.astype(np.float16).view(np.uint16)
    out = np.zeros((rows, OL.row_bytes(Q8, cols)), np.uint8)
    for r in range(rows):
        oracle.q8_quantize_row(OL.ptr(x[r]), OL.ptr(out[r]), cols)
    return out


def rand_weight(oracle, rng, dtype, rows, cols):
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    if dtype == F16:
        return w.astype(np.float16).view(np.uint16)
    out = np.zeros((rows, OL.row_bytes(dtype, cols)), np.uint8)
    fn = oracle.q8_quantize_weights if dtype == Q8 else oracle.q4_quantize_weights
    fn(OL.ptr(w), rows * cols // 32, OL.ptr(out))
    return out


# (activation dtype, weight dtype, K, N, rows, start): each pair's second
# call is smaller than its first
CALLS = {
    "q8": [(Q8, Q4, 2048, 5632, 64, 0), (Q8, Q4, 2048, 2048, 3, 1)],
    "f16": [(F16, F16, 2048, 2048, 24, 0), (F16, F16, 256, 1000, 1, 0)],
}


@pytest.mark.parametrize("kind", list(CALLS))
def test_matmul_noalloc_matches_matmul(gpu, oracle, kind):
    L = gpu.lib()
    fn = L.nc_matmul_2d_noalloc
    fn.restype, fn.argtypes = C.c_int, [C.c_void_p] * 3 + [C.c_int, C.c_int, C.c_void_p]
    rng = np.random.default_rng(len(kind))
    for adt, wdt, K, N, rows, start in CALLS[kind]:
        x = rand_act(oracle, rng, adt, rows, K)
        w = rand_weight(oracle, rng, wdt, N, K)
        dx, dw = DevAct(x, adt, rows, K), DevWeight(w, wdt, N, K)
        a, b = DevAct.empty(adt, rows, N), DevAct.empty(adt, rows, N)
        gpu.check(L.nc_matmul_2d(C.byref(dx.t), C.byref(dw.t), C.byref(a.t), start, rows, None), "matmul_2d")
        gpu.check(fn(C.byref(dx.t), C.byref(dw.t), C.byref(b.t), start, rows, None), "matmul_2d_noalloc")
        sync()
        want = np.zeros((rows, OL.row_bytes(adt, N)), np.uint8)
        oracle.matmul(OL.ptr(x), adt, OL.ptr(w), wdt, OL.ptr(want), adt, K, N, start, rows, None)
        got_a, got_b = a.ref()[start:], b.ref()[start:]
        assert np.array_equal(got_b, got_a), f"{kind} K={K} N={N}: noalloc differs from matmul_2d"
        assert np.array_equal(got_b, want[start:]), f"{kind} K={K} N={N}: noalloc differs from the oracle"


def test_matmul_noalloc_refuses_oversize(gpu, oracle):
    L = gpu.lib()
    fn = L.nc_matmul_2d_noalloc
    fn.restype, fn.argtypes = C.c_int, [C.c_void_p] * 3 + [C.c_int, C.c_int, C.c_void_p]
    rng = np.random.default_rng(5)
    K, N, rows = 256, 32768, 65  # 65 x 32768 x 4 bytes > 8 MiB
    x = rand_act(oracle, rng, Q8, rows, K)
    w = rand_weight(oracle, rng, Q8, N, K)
    dx, dw = DevAct(x, Q8, rows, K), DevWeight(w, Q8, N, K)
    out = DevAct.empty(Q8, rows, N)
    assert fn(C.byref(dx.t), C.byref(dw.t), C.byref(out.t), 0, rows, None) == -1
    assert "staging" in L.nc_last_error().decode()
