"""Pin the decoder-block pieces of the CPU oracle (oracle/catena_oracle_block.c)
against the reference's own tests, closed forms and libm, before they check
the GPU kernels."""
import json
import math
import os
import struct

import numpy as np

import oracle

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_known_answers.json")))


def bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def test_sqrt_newton_closed_forms_and_range():
    s = lambda x: oracle.scalar("sqrt_newton", x)  # noqa: E731
    assert s(1.0) == 1.0 and s(4.0) == 2.0 and s(0.25) == 0.5
    assert bits(s(0.0)) == 0 and bits(s(-3.0)) == 0  # non-positive -> +0
    for x in np.linspace(0.05, 60.0, 2001):
        assert abs(s(x) - math.sqrt(x)) <= 2e-7 * math.sqrt(x), x
    # six Newton steps from guess0 = x do not reach sqrt for large x
    # (catena-lang/stdlib/math.hex:235-272): a dropped step or a different
    # starting guess changes these values
    assert abs(s(1e6) - 15646.322) < 0.01

    def newton6(x):  # the same six steps in float64
        g = 1.0 if x < 1.0 else x
        for _ in range(6):
            g = 0.5 * (g + x / g)
        return g
    for x in [100.0, 250.0, 1e-3, 3e-5, 5e3]:
        assert abs(s(x) - newton6(x)) <= 1e-5 * newton6(x), x


def test_sigmoid_silu():
    c0 = struct.unpack("<f", struct.pack("<I", 0x3F7FF8FC))[0]
    # exp~(-0) = c0, so sigmoid(0) = 1 / (1 + c0) in f32
    expect = np.float32(1.0) / (np.float32(1.0) + np.float32(c0))
    assert bits(oracle.scalar("sigmoid", 0.0)) == bits(float(expect))
    for x in np.linspace(-12, 12, 481):
        sg = 1.0 / (1.0 + math.exp(-x))
        assert abs(oracle.scalar("sigmoid", x) - sg) < 0.014 * max(sg, 1e-3) + 1e-7
        assert abs(oracle.scalar("silu", x) - x * sg) < 0.014 * abs(x) * sg + 1e-6
    # silu = x * sigmoid(x) with one rounding
    for x in [-3.5, -0.1, 0.7, 2.25, 9.0]:
        expect = np.float32(x) * np.float32(oracle.scalar("sigmoid", x))
        assert bits(oracle.scalar("silu", x)) == bits(float(expect))


def test_sin_cos_full():
    assert oracle.scalar("sin_full", 0.0) == 0.0
    assert oracle.scalar("cos_full", 0.0) == 1.0
    xs = np.linspace(-100, 100, 20001).astype(np.float32)
    for x in xs[::7]:
        assert abs(oracle.scalar("sin_full", x) - math.sin(x)) < 1e-5, x
        assert abs(oracle.scalar("cos_full", x) - math.cos(x)) < 1e-5, x
    for x in [0.3, 1.7, 5.5, 42.0, 99.9]:
        assert bits(oracle.scalar("sin_full", -x)) == bits(-oracle.scalar("sin_full", x))
        assert bits(oracle.scalar("cos_full", -x)) == bits(oracle.scalar("cos_full", x))
    # the Taylor pieces themselves (reduced range)
    for r in np.linspace(-0.785, 0.785, 301):
        assert abs(oracle.scalar("sin_approx", r) - math.sin(r)) < 4e-7
        assert abs(oracle.scalar("cos_approx", r) - math.cos(r)) < 4e-6


def test_rmsnorm_reference_test():
    # catena-lang/tests/runtime.rs:1011-1044
    x = np.array([1.0, 2.0, 4.0, -1.0, -9.0, 13.29], np.float32)
    y = oracle.rmsnorm_f32(x)
    ms = float(np.mean(x.astype(np.float32) ** 2))
    rms = math.sqrt(ms + 1e-5)
    assert np.abs(y - x / rms).max() < 3e-3
    assert abs(math.sqrt(float(np.mean(y.astype(np.float64) ** 2))) - 1.0) < 3e-3
    # composition: y = x / sqrt_newton(fold(x*x)/n + eps)
    s = np.float32(0.0)
    for v in x:
        s = np.float32(s + np.float32(v * v))
    t = np.float32(np.float32(s / np.float32(len(x))) + np.float32(struct.unpack("<f", struct.pack("<I", 0x3727C5AC))[0]))
    rms_o = np.float32(oracle.scalar("sqrt_newton", float(t)))
    assert np.array_equal((x / rms_o).astype(np.float32).view(np.uint32), y.view(np.uint32))


def test_argmax_reference_cases():
    for values, expect in GOLDEN["argmax_first_index"]["cases"]:
        assert oracle.argmax_f32(np.array(values, np.float32)) == expect
    assert oracle.argmax_f32(np.array([1.0, np.nan, 0.5, 0.7], np.float32)) == 3
    assert oracle.argmax_f32(np.array([1.0, 2.0, np.nan], np.float32)) == 2
    assert oracle.argmax_f32(np.array([-np.inf, -np.inf], np.float32)) == 0


def test_rope():
    inv = oracle.rope_inv_freq(128, 10000.0)
    assert inv[0] == 1.0 and abs(inv[1] - 10000 ** (-2 / 128)) < 1e-7
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, 128).astype(np.float32)
    assert np.array_equal(oracle.rope_f32(x, 0, inv).view(np.uint32), x.view(np.uint32))
    for pos in [1, 17, 511, 639]:
        y = oracle.rope_f32(x, pos, inv).astype(np.float64)
        th = np.float32(pos) * inv.astype(np.float64)
        c, s = np.cos(th), np.sin(th)
        x1, x2 = x[:64].astype(np.float64), x[64:].astype(np.float64)
        assert np.abs(y[:64] - (x1 * c - x2 * s)).max() < 2e-4
        assert np.abs(y[64:] - (x2 * c + x1 * s)).max() < 2e-4
        n0 = x1 ** 2 + x2 ** 2
        n1 = y[:64] ** 2 + y[64:] ** 2
        assert np.abs(n1 - n0).max() < 1e-4 * (1 + n0.max())


def test_silu_mul_group_layout():
    """The interleaved layout is a permutation of the gate | up layout."""
    from oracle import decoder as od
    rng = np.random.default_rng(4)
    F, G = 256, 64
    g = rng.standard_normal((3, F)).astype(np.float32)
    u = rng.standard_normal((3, F)).astype(np.float32)
    halves = np.concatenate([g, u], axis=1)
    inter = np.concatenate([np.concatenate([g[:, i:i + G], u[:, i:i + G]], axis=1)
                            for i in range(0, F, G)], axis=1)
    assert np.array_equal(od.silu_mul_bf16(halves, F), od.silu_mul_bf16(inter, F, G))


def test_row_forms_equal_the_elementwise_composition():
    """The whole-activation oracle forms (or_silu_mul_rows, or_rope_qkv_rows,
    or_rmsnorm_rows) equal the pinned per-element / per-head / per-row
    functions they are built from, on both SwiGLU layouts, with specials in
    the gate / up columns and with positions that clamp at 0: a wrong gate /
    up index, head offset, position or row stride fails here."""
    from oracle import decoder as od
    rng = np.random.default_rng(9)
    rows, F = 5, 192
    gu = rng.standard_normal((rows, 2 * F)).astype(np.float32) * 4
    gu[0, 3] = np.nan
    gu[1, 70] = np.inf
    gu[2, 200] = -np.inf
    gu[3, :] = 0.0
    gu[4, 100] = 95.0   # exp~ of -95: the garbage range of the reference's exp
    for group in (0, 64, 32):
        a = od.silu_mul_bf16(gu, F, group)
        b = od.silu_mul_bf16_elementwise(gu, F, group)
        assert a.shape == (rows, F)
        an, bn = (a & 0x7FFF) > 0x7F80, (b & 0x7FFF) > 0x7F80
        assert np.array_equal(an, bn) and np.array_equal(a[~an], b[~bn]), group
    B, tq, H, Dh = 2, 3, 3, 128
    inv = oracle.rope_inv_freq(Dh, 10000.0)
    qkv = rng.standard_normal((B * tq, 3 * H * Dh)).astype(np.float32)
    # the second: sequences shorter than tq rotate at position 0; the third:
    # positions past a 4-position cache rotate at 0
    for lens, max_len in (([3, 700], None), ([1, 2], None), ([3, 6], 4)):
        fast = od.rope_qkv(qkv, inv, lens, B, tq, H, Dh, max_len=max_len)
        slow = od.rope_qkv_per_head(qkv, inv, lens, B, tq, H, Dh, max_len=max_len)
        for x, y in zip(fast, slow):
            assert np.array_equal(x, y)
    x = rng.standard_normal((4, 300)).astype(np.float32)
    want = np.stack([oracle.rmsnorm_f32(r) for r in x])
    assert np.array_equal(oracle.rmsnorm_f32(x).view(np.uint32), want.view(np.uint32))


def test_scalar_programs_reference_vectors():
    """The reference's own tests of the scalar programs (inputs, expected
    libm values and tolerances as fixtures, each citing its test):
    math.sin-approx, math.sin-approx-full, nn.sigmoid, nn.silu, math.sqrt."""
    for key, name in [("sin_approx", "sin_approx"), ("sin_approx_full", "sin_full"),
                      ("sigmoid", "sigmoid"), ("silu", "silu"), ("sqrt", "sqrt_newton")]:
        g = GOLDEN[key]
        got = oracle.map_f32(name, np.array(g["inputs"], np.float32))
        err = np.abs(got.astype(np.float64) - np.array(g["expected"], np.float64))
        assert np.all(err < g["absolute_tolerance"]), (key, float(err.max()))
