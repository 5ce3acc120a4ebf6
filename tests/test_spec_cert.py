"""The certificate that lets a speculative rms_norm launch keep a block of its
speculative row without requantizing it under the exact denominator.

A launch normalizes the row with a predicted denominator Ds while the exact
sum of squares (and so De) is still running, quantizes it to Q8 blocks
(gten/quants.cpp:16-30: absmax, delta = absmax / 127, fp16 delta, scale =
1 / delta, roundf) and later keeps every block the certificate covers:

* the codes of a block are invariant under a change of denominator up to
  14.0001 units in the last place of each scaled value z (the common factor
  cancels in z = y / (absmax / 127)), so a block whose every |z| is farther
  than 2^-20 |z| from a half-integer keeps its codes for any De;
* its fp16 delta keeps its value when the fp16 rounding is constant over
  dl * RN(Ds / De) * [1 - 10u, 1 + 10u].

The arithmetic below is the kernel's (`quad_quantize_cert`,
`spec_rms_chunk_cert`, `spec_rms_uncertain` in nc_dmv.h) in float32 numpy.
Denominators are planted wrong on purpose, from a few ulps to a factor of
two; every certified block must equal the exact one, bit for bit.  A
certificate with too tight a bound must fail the same check (the test can
see a wrong bound)."""
import numpy as np
import pytest

F = np.float32
U = 2.0 ** -24


def roundf(z):
    """C roundf: halves away from zero (as the kernel's round of z)."""
    t = np.trunc(z)
    return np.where(np.abs(z - t) >= F(0.5), t + np.copysign(F(1), z), t).astype(F)


def quantize(y):
    """Q8 blocks of y [B, 32]: codes, fp16 delta bits, fp32 delta, scaled values."""
    a = np.max(np.abs(y), axis=1)
    dl = (a / F(127)).astype(F)
    with np.errstate(divide="ignore"):
        scale = np.where(dl != 0, F(1) / dl, F(0)).astype(F)
    z = (y * scale[:, None]).astype(F)
    return roundf(z), dl.astype(np.float16).view(np.uint16), dl, z


def code_flags(z, bound=F(2.0 ** -20)):
    az = np.abs(z)
    return np.any(np.abs((az - np.floor(az)) - F(0.5)) <= az * bound, axis=1)


def norm_blocks(h, g, d, post):
    """The normalized row's final Q8 blocks, and the first quantization's
    (codes, fp16 delta, fp32 delta, scaled values) that the certificate reads."""
    y = (h / d * g).astype(F)
    first = quantize(y)
    if post != 1.0:
        q, d16 = first[0], first[1]
        y = (q * d16.view(np.float16).astype(F)[:, None]).astype(F)
        y = (y * F(post)).astype(F)
        q2, d162, _, _ = quantize(y)
        return (q2, d162), first
    return (first[0], first[1]), first


def uncertain(dl, flags, r):
    p = (dl * r).astype(F)
    lo = (p * F(1 - 10 * U)).astype(F)
    hi = (p * F(1 + 10 * U)).astype(F)
    d16 = dl.astype(np.float16)
    with np.errstate(invalid="ignore"):
        small = ~(dl >= F(2.0 ** -66))
    return flags | small | (lo.astype(np.float16) != d16) | (hi.astype(np.float16) != d16)


def rows(rng, nrows, K=2048):
    """Residual-stream-like rows: Q8 codes times fp16 deltas (some rows with
    outliers), and fp16 gains."""
    codes = rng.integers(-127, 128, (nrows, K)).astype(F)
    deltas = np.repeat(np.float16(rng.uniform(1e-4, 0.05, (nrows, K // 32))).astype(F), 32, axis=1)
    h = (codes * deltas).astype(F)
    out = rng.random(nrows) < 0.2
    h[out, :: 97] *= F(40)
    g = np.float16(rng.normal(1.0, 0.3, K)).astype(F)
    g[:: 13] = np.float16(rng.uniform(0.001, 4, len(g[:: 13])))
    return h, g


def exact_denom(h):
    ss = np.zeros(h.shape[0], F)
    for i in range(h.shape[1]):  # left to right, as the kernel's exact sum
        ss = (ss + h[:, i] * h[:, i]).astype(F)
    return (np.sqrt((ss / F(h.shape[1])).astype(F)) + F(1e-6)).astype(F)


RATIOS = [1 + k * U for k in (-37, -8, -3, -1, 1, 2, 5, 12, 40)] + [1 - 3e-5, 1 + 1e-3, 0.5, 2.0, 1.37]


def run(rng, post, bound=F(2.0 ** -20), nrows=256):
    h, g = rows(rng, nrows)
    de = exact_denom(h)
    K = h.shape[1]
    hb = h.reshape(-1, 32)
    gb = np.tile(g.reshape(-1, 32), (nrows, 1))
    deb = np.repeat(de, K // 32)
    stats = dict(blocks=0, uncertain=0, differ=0, wrong=0)
    (qe, de16), _ = norm_blocks(hb, gb, deb[:, None], post)
    for ratio in RATIOS:
        dsb = (deb * F(ratio)).astype(F)
        (qs, ds16), (_, _, dl, z) = norm_blocks(hb, gb, dsb[:, None], post)
        r = (dsb / deb).astype(F)
        unc = uncertain(dl, code_flags(z, bound), r)
        same = np.all(qs == qe, axis=1) & (ds16 == de16)
        stats["blocks"] += len(same)
        stats["uncertain"] += int(unc.sum())
        stats["differ"] += int((~same).sum())
        stats["wrong"] += int((~unc & ~same).sum())
    return stats


@pytest.mark.parametrize("post", [1.0, 1.4])
def test_certified_blocks_equal_the_exact_ones(post):
    s = run(np.random.default_rng(11 if post == 1.0 else 12), post)
    assert s["wrong"] == 0, s
    # the planted denominators did change blocks, and the certificate caught them all
    assert s["differ"] > 100, s
    # and it keeps most blocks (the kernel requantizes the rest)
    assert s["uncertain"] < 0.35 * s["blocks"], s


def test_too_tight_a_bound_is_seen():
    """The same check with a bound of half an ulp instead of 16: some block
    the weaker certificate keeps differs from the exact one."""
    s = run(np.random.default_rng(13), 1.0, bound=F(2.0 ** -25))
    assert s["wrong"] > 0, s


def test_same_denominator_same_row():
    """Ds == De: the rows are the same bit for bit (the kernel keeps them all)."""
    rng = np.random.default_rng(14)
    h, g = rows(rng, 32)
    de = exact_denom(h)
    hb = h.reshape(-1, 32)
    gb = np.tile(g.reshape(-1, 32), (32, 1))
    deb = np.repeat(de, 64)[:, None]
    a, _ = norm_blocks(hb, gb, deb, 1.0)
    b, _ = norm_blocks(hb.copy(), gb.copy(), deb.copy(), 1.0)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
