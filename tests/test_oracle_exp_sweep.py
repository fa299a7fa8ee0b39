"""Pin or_exp_approx bit for bit against a second, independent transcription.

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
"""
import concurrent.futures as cf
import os

import numpy as np

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
