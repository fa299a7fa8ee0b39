"""Pin the scalar oracle functions bit for bit against second, independent
transcriptions.

The second transcription below restates math.exp-approx-nonneg and
math.exp-approx (catena-lang/stdlib/math.hex:148-199) in numpy float32:
each hexpr node is one numpy operation on float32 / uint64 arrays (numpy's
float32 ufuncs are single IEEE operations, rounded to nearest even and never
fused), `f32.round-to-u32` is np.rint (ties to even) followed by the device's
saturating conversion (NaN and non-positive -> 0, >= 2^32 -> 0xFFFFFFFF), and
the u32 add and multiply wrap modulo 2^32.  It shares no code with the C
oracle, so a one-ulp slip in a constant, a ties-away rounding or a reordered
polynomial in either one fails the comparison.

Inputs: every one of the 2^32 float32 bit patterns, in chunks spread over
threads (numpy and the C oracle both release the GIL on whole arrays).

The other scalar programs (math.sqrt, nn.sigmoid, nn.silu, math.sin-approx,
math.cos-approx, math.sin-approx-full: catena-lang/stdlib/math.hex:1-103,
:235-272, catena-lang/stdlib/nn.hex:1-21) get the same kind of numpy
transcription, compared with the C oracle over 2^22 random bit patterns plus
2^23 evenly strided float32 values (each sign) over each one's working range.
"""
import concurrent.futures as cf
import os

import numpy as np
import pytest

import oracle


def _c(bits: int) -> np.float32:
    return np.array([bits], np.uint32).view(np.float32)[0]


INV_LN2, LN2_HI, LN2_LO = _c(0x3FB8AA3B), _c(0x3F317200), _c(0x35BFBE8E)
C0, C1, C2, C3 = _c(0x3F7FF8FC), _c(0x3F809C7E), _c(0x3EEF1187), _c(0x3E738A8B)
ONE = _c(0x3F800000)
ZERO = np.float32(0)


def _ties_away(v: np.ndarray) -> np.ndarray:
    return np.copysign(np.floor(np.abs(v) + np.float32(0.5)), v).astype(np.float32)


def exp_approx_numpy(x: np.ndarray, c1=None, ln2_lo=None, rounding=np.rint) -> np.ndarray:
    """math.exp-approx over a float32 array, one numpy op per hexpr node.
    c1, ln2_lo and rounding exist only so a test can plant a mistake."""
    c1 = C1 if c1 is None else c1
    ln2_lo = LN2_LO if ln2_lo is None else ln2_lo
    x = np.asarray(x, np.float32)
    with np.errstate(all="ignore"):
        # math.exp-approx: magnitude = (x < 0) ? -x : x
        is_negative = x < ZERO
        magnitude = np.where(is_negative, np.negative(x), x).astype(np.float32)
        # math.exp-approx-nonneg
        scaled = np.multiply(magnitude, INV_LN2, dtype=np.float32)
        rounded = rounding(scaled)  # np.rint: ties to even, still float32
        r64 = rounded.astype(np.float64)
        k = np.where(np.isnan(r64) | (r64 <= 0.0), 0.0,
                     np.where(r64 >= 4294967296.0, 4294967295.0, r64)).astype(np.uint64)
        k_f32 = k.astype(np.float32)  # exact below 2^24, one rounding above
        k_ln2_hi = np.multiply(k_f32, LN2_HI, dtype=np.float32)
        k_ln2_lo = np.multiply(k_f32, ln2_lo, dtype=np.float32)
        r1 = np.subtract(magnitude, k_ln2_hi, dtype=np.float32)
        xr = np.subtract(r1, k_ln2_lo, dtype=np.float32)
        xr_c3 = np.multiply(xr, C3, dtype=np.float32)
        p2 = np.add(C2, xr_c3, dtype=np.float32)
        xr_p2 = np.multiply(xr, p2, dtype=np.float32)
        p1 = np.add(c1, xr_p2, dtype=np.float32)
        xr_p1 = np.multiply(xr, p1, dtype=np.float32)
        poly = np.add(C0, xr_p1, dtype=np.float32)
        biased = (k + np.uint64(0x7F)) & np.uint64(0xFFFFFFFF)
        pow2_bits = (biased * np.uint64(0x00800000)) & np.uint64(0xFFFFFFFF)
        pow2k = pow2_bits.astype(np.uint32).view(np.float32)
        base = np.multiply(poly, pow2k, dtype=np.float32)
        reciprocal = np.divide(ONE, base, dtype=np.float32)
        return np.where(is_negative, reciprocal, base).astype(np.float32)


def _same_bits(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Equal bits, with any NaN equal to any NaN (payloads are not pinned)."""
    ua, ub = a.view(np.uint32), b.view(np.uint32)
    return (ua == ub) | (np.isnan(a) & np.isnan(b))


def _mismatches(start: int, count: int) -> tuple[int, list[int]]:
    x = np.arange(start, start + count, dtype=np.uint64).astype(np.uint32).view(np.float32)
    want = exp_approx_numpy(x)
    got = oracle.exp_approx_vec(x)
    bad = np.flatnonzero(~_same_bits(got, want))
    return bad.size, [int(x.view(np.uint32)[i]) for i in bad[:4]]


def test_numpy_transcription_known_points():
    # the closed forms the reference's arithmetic fixes, through the numpy form
    x = np.array([0.0, -0.0, 88.5, -89.5, np.nan], np.float32)
    y = exp_approx_numpy(x).view(np.uint32)
    assert y[0] == 0x3F7FF8FC and y[1] == 0x3F7FF8FC  # k = 0, r = 0: c0
    assert y[2] == 0x7F800000  # k = 128: 2^k is +inf
    assert y[3] == 0xFF800000  # k = 129 wraps to -0: 1 / -0 = -inf
    assert np.isnan(exp_approx_numpy(x)[4])


def test_exp_approx_bitwise_all_2_32_inputs():
    chunk = 1 << 22
    starts = range(0, 1 << 32, chunk)
    workers = max(1, min(8, len(os.sched_getaffinity(0))))
    total, examples = 0, []
    with cf.ThreadPoolExecutor(workers) as pool:
        for n_bad, ex in pool.map(lambda s: _mismatches(s, chunk), starts):
            total += n_bad
            examples += ex
    assert total == 0, f"{total} mismatching inputs, e.g. {[hex(b) for b in examples[:8]]}"


def test_mistakes_are_caught():
    """The comparison is sharp enough: each planted slip below (on the numpy
    side only) differs from the oracle somewhere in a small dense sweep."""
    x = np.linspace(-100, 100, 400_001, dtype=np.float32)
    good = oracle.exp_approx_vec(x)
    assert np.all(_same_bits(good, exp_approx_numpy(x)))
    assert not np.all(_same_bits(good, exp_approx_numpy(x, c1=_c(0x3F809C7F))))
    # k * ln2_lo only moves xr across a rounding boundary now and then: every
    # float32 from 64.0 up (k ~ 92..) for 2^22 patterns, both signs (58 of
    # the 8M inputs differ)
    xd = np.arange(0x42800000, 0x42800000 + (1 << 22), dtype=np.uint32).view(np.float32)
    xd = np.concatenate([xd, -xd])
    good_d = oracle.exp_approx_vec(xd)
    assert np.all(_same_bits(good_d, exp_approx_numpy(xd)))
    assert not np.all(_same_bits(good_d, exp_approx_numpy(xd, ln2_lo=_c(0x35BFBE8F))))
    # ties away from zero instead of ties to even: inputs whose x / ln2 is
    # exactly k + 1/2 (scaled below by a power of two, so exact in f32)
    xt = ((np.arange(0, 64, dtype=np.float32) + np.float32(0.5))
          / INV_LN2).astype(np.float32)
    xt = np.concatenate([xt, -xt])
    scaled = np.multiply(np.abs(xt), INV_LN2, dtype=np.float32)
    assert np.any(np.rint(scaled) != _ties_away(scaled))  # the sweep hits exact ties
    good_t = oracle.exp_approx_vec(xt)
    assert np.all(_same_bits(good_t, exp_approx_numpy(xt)))
    assert not np.all(_same_bits(good_t, exp_approx_numpy(xt, rounding=_ties_away)))


# ---------------------------------------------------------------- other scalar programs
HALF = _c(0x3F000000)
INV_PIO2, PIO2_HI, PIO2_LO = _c(0x3F22F983), _c(0x3FC90FDA), _c(0x33A22168)


def _round_to_u32(v: np.ndarray) -> np.ndarray:
    """f32.round-to-u32 with the device conversion, as uint64."""
    r64 = np.rint(v).astype(np.float64)
    return np.where(np.isnan(r64) | (r64 <= 0.0), 0.0,
                    np.where(r64 >= 4294967296.0, 4294967295.0, r64)).astype(np.uint64)


def sqrt_numpy(x, steps=6):
    """math.sqrt, catena-lang/stdlib/math.hex:235-272."""
    x = np.asarray(x, np.float32)
    with np.errstate(all="ignore"):
        g = np.where(x < ONE, ONE, x).astype(np.float32)
        for _ in range(steps):
            ratio = np.divide(x, g, dtype=np.float32)
            g = np.multiply(np.add(g, ratio, dtype=np.float32), HALF, dtype=np.float32)
        return np.where(x <= ZERO, ZERO, g).astype(np.float32)


def sigmoid_numpy(x):
    """nn.sigmoid, catena-lang/stdlib/nn.hex:1-12: 1 / (1 + exp~(-x))."""
    x = np.asarray(x, np.float32)
    with np.errstate(all="ignore"):
        den = np.add(ONE, exp_approx_numpy(np.negative(x)), dtype=np.float32)
        return np.divide(ONE, den, dtype=np.float32)


def silu_numpy(x):
    """nn.silu, catena-lang/stdlib/nn.hex:15-21: x * sigmoid(x)."""
    x = np.asarray(x, np.float32)
    with np.errstate(all="ignore"):
        return np.multiply(x, sigmoid_numpy(x), dtype=np.float32)


def sin_taylor_numpy(x):
    """math.sin-approx, catena-lang/stdlib/math.hex:1-23."""
    x = np.asarray(x, np.float32)
    with np.errstate(all="ignore"):
        x2 = np.multiply(x, x, dtype=np.float32)
        x3 = np.multiply(x2, x, dtype=np.float32)
        x5 = np.multiply(x3, x2, dtype=np.float32)
        x7 = np.multiply(x5, x2, dtype=np.float32)
        a = np.divide(x3, np.float32(6), dtype=np.float32)
        b = np.divide(x5, np.float32(120), dtype=np.float32)
        c = np.divide(x7, np.float32(5040), dtype=np.float32)
        return np.subtract(np.add(np.subtract(x, a, dtype=np.float32), b, dtype=np.float32), c,
                           dtype=np.float32)


def cos_taylor_numpy(x):
    """math.cos-approx, catena-lang/stdlib/math.hex:25-47."""
    x = np.asarray(x, np.float32)
    with np.errstate(all="ignore"):
        x2 = np.multiply(x, x, dtype=np.float32)
        x4 = np.multiply(x2, x2, dtype=np.float32)
        x6 = np.multiply(x4, x2, dtype=np.float32)
        a = np.divide(x2, np.float32(2), dtype=np.float32)
        b = np.divide(x4, np.float32(24), dtype=np.float32)
        c = np.divide(x6, np.float32(720), dtype=np.float32)
        return np.subtract(np.add(np.subtract(ONE, a, dtype=np.float32), b, dtype=np.float32), c,
                           dtype=np.float32)


def sin_full_numpy(x, quadrant_order=(0, 1, 2)):
    """math.sin-approx-full(-nonneg), catena-lang/stdlib/math.hex:49-103.
    quadrant_order exists only so a test can plant a mistake."""
    x = np.asarray(x, np.float32)
    with np.errstate(all="ignore"):
        is_negative = x < ZERO
        mag = np.where(is_negative, np.negative(x), x).astype(np.float32)
        n_u32 = _round_to_u32(np.multiply(mag, INV_PIO2, dtype=np.float32))
        n_f = n_u32.astype(np.float32)
        r1 = np.subtract(mag, np.multiply(n_f, PIO2_HI, dtype=np.float32), dtype=np.float32)
        r = np.subtract(r1, np.multiply(n_f, PIO2_LO, dtype=np.float32), dtype=np.float32)
        sin_r, cos_r = sin_taylor_numpy(r), cos_taylor_numpy(r)
        quadrant = n_u32 & np.uint64(3)
        q0, q1, q2 = quadrant_order
        q23 = np.where(quadrant == q2, np.negative(sin_r), np.negative(cos_r))
        q123 = np.where(quadrant == q1, cos_r, q23)
        base = np.where(quadrant == q0, sin_r, q123).astype(np.float32)
        return np.where(is_negative, np.negative(base), base).astype(np.float32)


_SCALAR = {
    # name: (numpy transcription, first float32 of the run (bits), binades);
    # the run takes every binades-th bit pattern from there, 2^23 values,
    # so it spans that many binades, both signs
    "sqrt_newton": (sqrt_numpy, 0x3A800000, 24),   # 2^-10 .. 2^14
    "sigmoid": (sigmoid_numpy, 0x3C000000, 14),    # 2^-7 .. 2^7
    "silu": (silu_numpy, 0x3C000000, 14),
    "sin_approx": (sin_taylor_numpy, 0x39800000, 13),  # 2^-12 .. 2
    "cos_approx": (cos_taylor_numpy, 0x39800000, 13),
    "sin_full": (sin_full_numpy, 0x3F000000, 10),  # 0.5 .. 512
}


def _scalar_inputs(first: int, binades: int) -> np.ndarray:
    rng = np.random.default_rng(first)
    rand = rng.integers(0, 1 << 32, 1 << 22, dtype=np.uint64).astype(np.uint32)
    run = (first + binades * np.arange(1 << 23, dtype=np.uint64)).astype(np.uint32)
    specials = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x00000001,
                         0x3F800000, 0xBF800000, 0x7F7FFFFF], np.uint32)
    u = np.concatenate([rand, run, run | np.uint32(0x80000000), specials])
    return u.view(np.float32)


@pytest.mark.parametrize("name", sorted(_SCALAR))
def test_scalar_oracle_bitwise_vs_numpy_transcription(name):
    fn, first, binades = _SCALAR[name]
    x = _scalar_inputs(first, binades)
    got = oracle.map_f32(name, x)
    want = fn(x)
    bad = np.flatnonzero(~_same_bits(got, want))
    assert bad.size == 0, (bad.size, [hex(int(v)) for v in x.view(np.uint32)[bad[:6]]])


def test_scalar_planted_mistakes_are_caught():
    """Each slip below (on the numpy side) differs from the oracle on the
    fixture's reference inputs or a small sweep."""
    x = np.linspace(-50, 50, 200_001, dtype=np.float32)
    assert not np.all(_same_bits(oracle.map_f32("sqrt_newton", np.abs(x)),
                                 sqrt_numpy(np.abs(x), steps=5)))
    assert not np.all(_same_bits(oracle.map_f32("sin_full", x),
                                 sin_full_numpy(x, quadrant_order=(0, 2, 1))))
    # sigmoid from the exact exponential instead of exp~
    exact = (ONE / (ONE + np.exp(-x.astype(np.float64)))).astype(np.float32)
    assert not np.all(_same_bits(oracle.map_f32("sigmoid", x), exact))
