"""The Q4 offset of the long-prompt prefill matmul, restated on the CPU.

The reference's Q4 block dot product (gten/ops.cpp:387-490) multiplies each
activation code x by the decoded weight n - 7 (n the stored nibble) and sums
eight such products per AVX lane.  The long-prompt shape of k_gemm_qh hands
the fp16 matrix cores the raw weight 1024 + n instead (fp16 bits 0x6400 | n,
one v_perm_b32 per two codes) and starts each product sum from
-1031 x (sum of the lane's activation codes).  That equals the reference's
integer lane sum exactly when every value the matrix core can form on the way
is an integer below 2^24 (exact in fp32 whatever the order of the adds).
These tests check that bound and the identity on random and extreme codes,
in several summation orders, and that a wrong offset is caught.
"""
import numpy as np
import pytest

rng = np.random.default_rng(20261203)


def _fp16_bits_to_float(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def _lane_sum_fp32(x, n, start, order):
    """Sum start + sum_i (1024 + n_i) * x_i in float32, adds in `order`."""
    w = _fp16_bits_to_float(0x6400 | n.astype(np.uint16))  # 1024 + n
    xv = x.astype(np.float16).astype(np.float32)  # codes -127..127, exact in fp16
    acc = np.float32(start)
    peak = abs(float(acc))
    for i in order:
        p = np.float32(w[i]) * np.float32(xv[i])
        peak = max(peak, abs(float(p)))
        acc = np.float32(acc + p)
        peak = max(peak, abs(float(acc)))
    return acc, peak


def _cases():
    out = []
    for _ in range(3000):
        out.append((rng.integers(-127, 128, 8), rng.integers(0, 16, 8)))
    # extremes: largest magnitudes of both signs, all-zero codes, mixed
    for xs in (127, -127, 0):
        for ns in (0, 15, 7):
            out.append((np.full(8, xs), np.full(8, ns)))
    out.append((np.array([127, -127] * 4), np.array([15, 0] * 4)))
    return out


def _orders():
    fwd = list(range(8))
    return [fwd, fwd[::-1], [0, 2, 4, 6, 1, 3, 5, 7]] + [list(rng.permutation(8)) for _ in range(3)]


def test_raw_fp16_codes_are_exact():
    for b in range(256):
        assert float(_fp16_bits_to_float(0x6400 | b)) == 1024.0 + b


@pytest.mark.parametrize("offset", [1031])
def test_offset_start_gives_the_reference_lane_sum(offset):
    worst = 0.0
    for x, n in _cases():
        want = int(np.sum((n.astype(np.int64) - 7) * x.astype(np.int64)))
        start = np.float32(-offset * int(np.sum(x)))
        for order in _orders():
            got, peak = _lane_sum_fp32(x, n, start, order)
            worst = max(worst, peak)
            assert float(got) == float(want), (x, n, order)
    # every product and partial sum is an integer below 2^24: exact in fp32
    assert worst < 2.0 ** 22


def test_a_wrong_offset_is_caught():
    # 1024 (forgetting the -7 of the decoded weight) must not pass
    bad = 0
    for x, n in _cases():
        want = int(np.sum((n.astype(np.int64) - 7) * x.astype(np.int64)))
        got, _ = _lane_sum_fp32(x, n, np.float32(-1024 * int(np.sum(x))), list(range(8)))
        bad += float(got) != float(want)
    assert bad > 2500
