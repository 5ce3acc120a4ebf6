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


# ---- layer_norm's mean: the left-to-right fp32 sum of signed fp16-grid values
# (gten/ops.cpp:673-676), computed from exact double prefixes and the few
# steps that round.

GRID_SIZES = [1024, 2048, 2304]


def grid_rows(n, rng):
    """Named rows of n signed values on the fp16 grid (fp16 activations and
    Q8 codes times fp16 deltas), some built to round often or to leave the
    grid (those must take the plain loop)."""
    out = {}
    f16 = lambda a: np.asarray(a, np.float16).astype(np.float32)
    out["f16_normal"] = f16(rng.standard_normal(n))
    out["f16_small"] = f16(rng.normal(0, 0.05, n))
    out["f16_heavy_tail"] = f16(rng.standard_t(3, n) * 0.3)
    out["f16_outliers"] = f16(np.where(rng.random(n) < 0.01, rng.normal(0, 300, n), rng.normal(0, 1, n)))
    out["f16_max"] = f16(np.where(rng.random(n) < 0.5, 65504.0, -65504.0) * (rng.random(n) < 0.1))
    out["f16_subnormal_mix"] = f16(np.where(rng.random(n) < 0.5, rng.normal(0, 1e-6, n), rng.normal(0, 50, n)))
    up = f16(np.abs(rng.normal(0, 1, n)))
    out["f16_growing"] = up  # the running sum grows through many binades
    alt = f16(rng.normal(0, 1, n))
    alt[::2] = 1000.0
    alt[1::2] = -1000.0 + alt[1::2] * 1e-3
    out["f16_cancelling"] = f16(alt)
    q = rng.integers(-127, 128, n).astype(np.float32)
    d = f16(rng.uniform(1e-3, 0.05, n // 32))
    out["q8_row"] = q * np.repeat(d, 32)
    out["zeros"] = np.zeros(n, np.float32)
    # a large value, a few small ones that round on its grid (ties to even
    # keep 1024; the mixed row rounds both ways), then small integers that
    # add exactly: the error carried from the rounding steps decides the
    # result
    ab = rng.integers(-3, 4, n).astype(np.float32)
    ab[0] = 1024.0
    ab[1:11] = 2.0 ** -14
    out["absorbed"] = ab
    mix = rng.integers(-3, 4, n).astype(np.float32)
    mix[0] = 1536.0
    mix[1:13] = f16(2.0 ** rng.integers(-16, -12, 12) * rng.choice([-3.0, -1.0, 1.0, 3.0], 12))
    out["absorbed_mixed"] = mix
    off = f16(rng.standard_normal(n))
    off[n // 2] = np.float32(3.0 * 2.0 ** -30)  # not a multiple of 2^-24: plain loop
    out["off_grid"] = off
    big = f16(rng.standard_normal(n))
    big[n // 3] = np.float32(2.0 ** 18)  # beyond the grid's range: plain loop
    out["too_large"] = big
    inf = f16(rng.standard_normal(n))
    inf[n // 4] = np.inf
    out["inf"] = inf
    return out


def grid_host(nc):
    f = nc.lib().nc_seq_sum_grid_host
    f.restype = C.c_float
    f.argtypes = [C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_int)]
    return f


@pytest.mark.parametrize("n", GRID_SIZES)
def test_grid_sum_host_equals_sequential_sum(nc, oracle, n):
    f = grid_host(nc)
    rng = np.random.default_rng(500 + n)
    passes = []
    for rep in range(10):
        for name, x in grid_rows(n, rng).items():
            x = np.ascontiguousarray(x, np.float32)
            want = oracle.seq_sum(x.ctypes.data_as(C.c_void_p), n)
            p = C.c_int()
            got = f(x.ctypes.data_as(C.c_void_p), n, 0, C.byref(p))
            assert same(got, want), (name, n, rep, got, want)
            if name in ("off_grid", "too_large", "inf"):
                assert p.value == 0, name  # the plain loop ran
            elif name.startswith("f16_normal"):
                passes.append(p.value)
    # realistic rows round at a few steps: a few passes each
    assert 1 <= np.mean(passes) <= 16, passes


def test_grid_sum_planted_mistake_is_caught(nc, oracle):
    """Dropping the rounding error after a rounding step (a planted mistake
    in the host run) must change results on these rows: the test above has
    teeth."""
    f = grid_host(nc)
    rng = np.random.default_rng(9)
    wrong = 0
    for rep in range(20):
        for name in ("absorbed", "absorbed_mixed"):
            x = np.ascontiguousarray(grid_rows(2048, rng)[name])
            want = oracle.seq_sum(x.ctypes.data_as(C.c_void_p), 2048)
            p = C.c_int()
            wrong += not same(f(x.ctypes.data_as(C.c_void_p), 2048, 1, C.byref(p)), want)
    assert wrong >= 20, wrong


@pytest.mark.gpu
@pytest.mark.parametrize("n", GRID_SIZES)
def test_grid_sum_device(gpu, oracle, n):
    L = gpu.lib()
    rng = np.random.default_rng(700 + n)
    names, rows = [], []
    for rep in range(60):
        for name, x in grid_rows(n, rng).items():
            names.append(name)
            rows.append(x)
    X = np.ascontiguousarray(np.stack(rows).astype(np.float32))
    cnt = X.shape[0]
    dx = dev_array(X)
    dout = NC.DeviceBuffer(cnt * 4)
    dpass = NC.DeviceBuffer(cnt * 4)
    NC.check(L.nc_block_seq_sum_grid(C.c_void_p(dx.ptr), n, cnt, C.c_void_p(dout.ptr), C.c_void_p(dpass.ptr), None))
    sync()
    out = np.zeros(cnt, np.float32)
    passes = np.zeros(cnt, np.int32)
    dout.download(out)
    dpass.download(passes)
    host = grid_host(gpu)
    bad = []
    for i in range(cnt):
        want = oracle.seq_sum(X[i].ctypes.data_as(C.c_void_p), n)
        hp = C.c_int()
        host(X[i].ctypes.data_as(C.c_void_p), n, 0, C.byref(hp))
        if not same(out[i], want) or passes[i] != hp.value:
            bad.append((i, names[i], float(out[i]), float(want), int(passes[i]), hp.value))
    assert not bad, bad[:5]
