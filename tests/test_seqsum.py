"""The exact parallel restatement of the reference's left-to-right fp32 sum
of non-negative terms (rms_norm's sum of squares, gten/ops.cpp:833-835).

The decomposition (binade segments as parity maps, crossings replayed) is
checked against the plain sequential loop of the oracle on vectors built to
break it: ties on the rounding grid, sums landing exactly on powers of two,
zeros and subnormals, huge dynamic ranges, infinities and NaNs.  The host run
also takes a skew that makes its binade predictions wrong on purpose: the
segment checks must then reject the segment (fast path off) or the result
must still be the sequential one."""
import ctypes as C

import numpy as np
import pytest

from devutil import dev_array, sync
from nc_pkg import nc as NC

SIZES = [1, 7, 256, 2048, 2304, 4096]


def vectors(n, rng):
    """Named float32 vectors of n non-negative terms."""
    out = {}
    q = rng.integers(-127, 128, n).astype(np.float32)
    d = np.float16(rng.uniform(1e-3, 0.05, n)).astype(np.float32)
    x = q * d
    out["q8_squares"] = x * x
    out["normal_squares"] = np.square(rng.standard_normal(n).astype(np.float32))
    out["small_ints_pow2"] = (rng.integers(0, 17, n) * 2.0 ** rng.integers(-3, 4, n)).astype(np.float32)
    out["ones"] = np.ones(n, np.float32)
    out["wide_range"] = (2.0 ** rng.uniform(-60, 60, n)).astype(np.float32)
    z = np.square(rng.standard_normal(n).astype(np.float32))
    z[: n // 2] = 0
    out["leading_zeros"] = z
    out["zeros"] = np.zeros(n, np.float32)
    one = np.zeros(n, np.float32)
    one[n // 3] = 3.5
    out["single"] = one
    sub = rng.integers(1, 1 << 23, n).astype(np.uint32).view(np.float32).copy()
    sub[::3] = np.float32(2.0 ** -125)
    out["subnormal"] = sub
    big = np.square(rng.standard_normal(n).astype(np.float32))
    big[n // 2] = 1e30
    out["huge_term"] = big
    out["geometric_up"] = (1.001 ** np.arange(n)).astype(np.float32)
    out["geometric_down"] = (0.997 ** np.arange(n)).astype(np.float32)
    # terms half a grid step of typical running sums (tie-heavy)
    out["half_ulps"] = (2.0 ** rng.integers(-24, -18, n) * 1024).astype(np.float32)
    out["near_pow2"] = np.full(n, np.float32(1.0) - np.float32(2.0 ** -24) * rng.integers(0, 4, n), np.float32)
    inf = np.square(rng.standard_normal(n).astype(np.float32))
    inf[n // 2] = np.inf
    out["inf"] = inf
    nan = np.square(rng.standard_normal(n).astype(np.float32))
    nan[n // 4] = np.nan
    out["nan"] = nan
    return out


def same(a, b):
    a, b = np.float32(a), np.float32(b)
    if np.isnan(a) or np.isnan(b):
        return bool(np.isnan(a) and np.isnan(b))
    return a.view(np.uint32) == b.view(np.uint32)


def host_fn(nc):
    f = nc.lib().nc_seq_sum_nonneg_host
    f.restype = C.c_float
    f.argtypes = [C.c_void_p, C.c_int, C.c_double, C.POINTER(C.c_int)]
    return f


@pytest.mark.parametrize("n", SIZES)
def test_host_decomposition_equals_sequential_sum(nc, oracle, n):
    f = host_fn(nc)
    rng = np.random.default_rng(n)
    fast_total = 0
    cases = 0
    for rep in range(20):
        for name, t in vectors(n, rng).items():
            t = np.ascontiguousarray(t, np.float32)
            want = oracle.seq_sum(t.ctypes.data_as(C.c_void_p), n)
            for skew in (0.0, 1e-7, -1e-7, 3e-5, -1e-3, 0.25):
                fast = C.c_int()
                got = f(t.ctypes.data_as(C.c_void_p), n, skew, C.byref(fast))
                assert same(got, want), (name, n, rep, skew, got, want)
                # near_pow2 keeps running sums within rounding of powers of
                # two on purpose: its predictions may fail (and fall back)
                if skew == 0.0 and name not in ("inf", "nan", "near_pow2"):
                    fast_total += fast.value
                    cases += 1
    # with exact predictions the parallel path must nearly always hold
    assert fast_total >= 0.95 * cases, (fast_total, cases)


def test_host_decomposition_skew_is_caught(nc, oracle):
    """Wrong binade predictions must never leak into the result: with a large
    skew most segments fail their check, and every result is still exact."""
    f = host_fn(nc)
    rng = np.random.default_rng(7)
    slow = 0
    for rep in range(200):
        t = np.square(rng.standard_normal(2048).astype(np.float32))
        want = oracle.seq_sum(t.ctypes.data_as(C.c_void_p), 2048)
        fast = C.c_int()
        got = f(t.ctypes.data_as(C.c_void_p), 2048, 0.25, C.byref(fast))
        assert same(got, want)
        slow += 1 - fast.value
    assert slow > 150


@pytest.mark.gpu
@pytest.mark.parametrize("n", [256, 2048, 2304, 4096])
def test_block_seq_sum_device(gpu, oracle, n):
    L = gpu.lib()
    rng = np.random.default_rng(100 + n)
    names, rows = [], []
    for rep in range(40):
        for name, t in vectors(n, rng).items():
            names.append(name)
            rows.append(t)
    # plus many realistic rows (the rms_norm inputs of the decode step)
    q = rng.integers(-127, 128, (4000, n)).astype(np.float32)
    d = np.float16(rng.uniform(1e-3, 0.05, (4000, n // 32))).astype(np.float32)
    x = q * np.repeat(d, 32, axis=1)
    for r in x * x:
        names.append("q8_rows")
        rows.append(r)
    T = np.ascontiguousarray(np.stack(rows).astype(np.float32))
    cnt = T.shape[0]
    dt = dev_array(T)
    dout = NC.DeviceBuffer(cnt * 4)
    dfast = NC.DeviceBuffer(cnt * 4)
    NC.check(L.nc_block_seq_sum(C.c_void_p(dt.ptr), n, cnt, C.c_void_p(dout.ptr), C.c_void_p(dfast.ptr), None))
    sync()
    out = np.zeros(cnt, np.float32)
    fast = np.zeros(cnt, np.int32)
    dout.download(out)
    dfast.download(fast)
    bad = []
    for i in range(cnt):
        want = oracle.seq_sum(T[i].ctypes.data_as(C.c_void_p), n)
        if not same(out[i], want):
            bad.append((i, names[i], float(out[i]), float(want), int(fast[i])))
    assert not bad, bad[:5]
    # the fallback (sequential loop) is exact too, only slower: the parallel
    # path must carry nearly all realistic rows (a thread's chunk may hold at
    # most four binade crossings; 16-term chunks at n = 4096 see more)
    real = [fast[i] for i in range(cnt) if names[i] == "q8_rows"]
    floor = 0.99 if n <= 2304 else 0.95
    assert sum(real) >= floor * len(real), f"parallel path taken for {sum(real)} of {len(real)} realistic rows"
