"""Pin the CPU oracle before trusting it as the checker.

Each oracle function is checked against (a) the reference's own known-answer
tests (tests/golden/reference_known_answers.json, each entry cites its
reference file), (b) closed forms of the reference's arithmetic, and (c)
independent computations (float64 / numpy float32 / torch) chosen so that a
plausible mistake -- a dropped term, a transposed operand, a wrong fold order
or a fused multiply-add -- fails at least one of them.
"""
import json
import math
import os
import struct

import numpy as np
import pytest

import oracle

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_known_answers.json")))


def bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def f32(b: int) -> float:
    return struct.unpack("<f", struct.pack("<I", b))[0]


# ---------------------------------------------------------------- matmul
def test_matmul_reference_known_answer():
    g = GOLDEN["matmul_2x2_via_mem"]
    a = np.array(g["a"], np.float32).reshape(g["n"], g["k"])
    b = np.array(g["b"], np.float32).reshape(g["k"], g["m"])
    c = oracle.matmul_f32(a, b)
    # the reference allows 1e-4; the values are exact in f32
    assert c.ravel().tolist() == g["expected"]


def test_matmul_identity_exact():
    g = GOLDEN["matmul_identity"]
    a = np.array(g["a"], np.float32).reshape(g["n"], g["n"])
    eye = np.eye(g["n"], dtype=np.float32)
    assert oracle.matmul_f32(a, eye).ravel().tolist() == g["expected"]
    assert oracle.matmul_f32(eye, a).ravel().tolist() == g["expected"]


def _seq_fold_numpy(a, b):
    """Independent float32 restatement: numpy's float32 ops are IEEE RNE and
    never fused, so this is the reference's per-cell fold order."""
    acc = np.zeros((a.shape[0], b.shape[1]), np.float32)
    for kk in range(a.shape[1]):
        prod = (a[:, kk:kk + 1] * b[kk:kk + 1, :]).astype(np.float32)
        acc = (acc + prod).astype(np.float32)
    return acc


@pytest.mark.parametrize("n,m,k", [(1, 1, 1), (3, 5, 7), (64, 48, 40), (33, 17, 129)])
def test_matmul_bitwise_vs_numpy_fold(n, m, k):
    rng = np.random.default_rng(n * 1000 + m * 10 + k)
    a = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, m)).astype(np.float32)
    c = oracle.matmul_f32(a, b)
    ref = _seq_fold_numpy(a, b)
    assert np.array_equal(c.view(np.uint32), ref.view(np.uint32))


def test_matmul_256_error_bound_and_not_transposed():
    rng = np.random.default_rng(1)
    a = rng.uniform(-1, 1, (256, 256)).astype(np.float32)
    b = rng.uniform(-1, 1, (256, 256)).astype(np.float32)
    c = oracle.matmul_f32(a, b).astype(np.float64)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    bound = 256 * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert np.all(np.abs(c - exact) <= bound)
    # a transposed operand or swapped index would be O(1) off
    wrong = a.astype(np.float64).T @ b.astype(np.float64)
    assert np.abs(c - wrong).max() > 1.0


def test_matmul_fold_is_not_fused():
    # single-cell k=2 case where a fused a*b + c differs from the rounded one
    # (the reference's own FMA example, catena-lang/tests/runtime.rs:333-363):
    # 1*c + a*b with acc = 0 + c first.
    a1, b1 = f32(0x3F800001), f32(0x3F800001)
    c = f32(0x33800000)
    A = np.array([[1.0, a1]], np.float32)
    B = np.array([[c], [b1]], np.float32)
    out = oracle.matmul_f32(A, B)[0, 0]
    # sequential: acc = 0 + 1*c = c; acc = c + fl(a1*b1)
    expect = np.float32(np.float32(c) + np.float32(np.float32(a1) * np.float32(b1)))
    assert bits(out) == bits(float(expect))


# ---------------------------------------------------------------- folds
def test_fold_known_answers():
    g = GOLDEN["sum_mean_max_f32"]
    x = np.array(g["input"], np.float32)
    assert oracle.fold_sum_f32(x) == g["sum"]
    assert oracle.fold_sum_f32(x) / len(x) == g["mean"]
    assert oracle.fold_max_f32(x) == g["max"]


def test_fold_max_semantics():
    # acc starts at -inf and keeps acc on ties: first of +0 / -0 wins
    assert bits(oracle.fold_max_f32(np.array([0.0, -0.0], np.float32))) == 0x00000000
    assert bits(oracle.fold_max_f32(np.array([-0.0, 0.0], np.float32))) == 0x80000000
    assert oracle.fold_max_f32(np.array([], np.float32)) == float("-inf")
    # a NaN resets the fold: the result is the max of what follows it
    x = np.array([5.0, np.nan, 1.0, 2.0], np.float32)
    assert oracle.fold_max_f32(x) == 2.0
    assert math.isnan(oracle.fold_max_f32(np.array([1.0, np.nan], np.float32)))


def test_fold_sum_order():
    # (1e8 + 1) - 1e8 == 0 in a left fold; a pairwise or reversed sum differs
    x = np.array([1e8, 1.0, -1e8, 1.0], np.float32)
    assert oracle.fold_sum_f32(x) == 1.0


# ---------------------------------------------------------------- exp~
def test_exp_approx_reference_tolerance():
    g = GOLDEN["exp_approx"]
    for x in g["inputs"]:
        y = oracle.exp_approx(x)
        e = math.exp(x)
        assert abs(y - e) / max(e, 1.0) < g["relative_tolerance"], x


def test_exp_approx_closed_forms():
    for case in GOLDEN["exp_approx_closed_form"]["cases"]:
        x = f32(int(case["x_bits"], 16)) if "x_bits" in case else case["x"]
        y = oracle.exp_approx(x)
        assert bits(y) == int(case["y_bits"], 16), case
    assert math.isnan(oracle.exp_approx(float("nan")))


def test_exp_approx_error_profile():
    """The cubic is accurate on the k=0 positive side (r in [0, ln2/2]) and
    reaches ~1.3% on the r < 0 side of each binade (the reference's own
    accuracy, not a bug here).  A dropped or wrong polynomial term, a wrong
    split-ln2 constant or a broken 2^k construction moves these bounds."""
    def max_rel(lo, hi, n):
        xs = np.linspace(lo, hi, n).astype(np.float32)
        ys = oracle.exp_approx_vec(xs).astype(np.float64)
        ex = np.exp(xs.astype(np.float64))
        return float((np.abs(ys - ex) / ex).max())
    assert max_rel(0.0, 0.3465, 4001) < 1.2e-4
    worst = max_rel(-87.0, 87.0, 60001)
    assert 1.2e-2 < worst < 1.4e-2
    # exp~(-x) is exactly 1/exp~(x) for x > 0 (the negative branch)
    for x in [0.1, 0.5, 1.0, 2.5, 10.0, 40.0]:
        assert bits(oracle.exp_approx(-x)) == bits(float(np.float32(1.0) / np.float32(oracle.exp_approx(x))))


def test_round_to_u32_device_semantics():
    L = oracle.lib()
    assert L.or_round_to_u32(2.5) == 2  # RNE
    assert L.or_round_to_u32(3.5) == 4
    assert L.or_round_to_u32(-1.0) == 0
    assert L.or_round_to_u32(float("nan")) == 0
    assert L.or_round_to_u32(5e9) == 0xFFFFFFFF


# ---------------------------------------------------------------- softmax
def test_softmax_reference_tolerance():
    g = GOLDEN["softmax"]
    x = np.array(g["input"], np.float32)
    y = oracle.softmax_f32(x)
    e = np.exp(x.astype(np.float64) - x.max())
    expect = e / e.sum()
    assert np.abs(y - expect).max() < g["absolute_tolerance"]
    assert abs(float(y.astype(np.float64).sum()) - 1.0) < g["sum_tolerance"]


def test_softmax_composition():
    # out_i = exp~(x_i - max) / fold_sum(exp~(x_j - max)), bit for bit
    rng = np.random.default_rng(7)
    x = rng.normal(0, 3, 257).astype(np.float32)
    y = oracle.softmax_f32(x)
    m = oracle.fold_max_f32(x)
    e = oracle.exp_approx_vec((x - np.float32(m)).astype(np.float32))
    den = np.float32(oracle.fold_sum_f32(e))
    assert np.array_equal((e / den).astype(np.float32).view(np.uint32), y.view(np.uint32))


def test_softmax_constant_and_single():
    y = oracle.softmax_f32(np.full(8, 3.0, np.float32))
    c0 = f32(0x3F7FF8FC)
    den = np.float32(0.0)
    for _ in range(8):
        den = np.float32(den + np.float32(c0))
    assert np.all(y == np.float32(np.float32(c0) / den))
    assert oracle.softmax_f32(np.array([123.0], np.float32))[0] == 1.0


# ---------------------------------------------------------------- bf16
def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.normal(0, 1, 20000).astype(np.float32),
        rng.normal(0, 1e30, 2000).astype(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-40, -1e-40], np.float32),
        np.array([f32(0x3F808000), f32(0x3F818000), f32(0x3F80FFFF), f32(0x7F7FFFFF)], np.float32),
    ])
    ours = oracle.f32_to_bf16_bits_np(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    # the scalar C routine agrees with the vectorised numpy one
    assert np.array_equal(oracle.f32_to_bf16(x[:3000]), ours[:3000])
    nan = oracle.f32_to_bf16(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


def test_bf16_gemm_integer_exact_and_bound():
    rng = np.random.default_rng(11)
    # small integers: every product and partial sum is exact
    ai = rng.integers(-8, 9, (19, 70)).astype(np.float32)
    bi = rng.integers(-8, 9, (70, 23)).astype(np.float32)
    ab, bb = oracle.f32_to_bf16_bits_np(ai), oracle.f32_to_bf16_bits_np(bi)
    c32, c16 = oracle.matmul_bf16(ab, bb)
    assert np.array_equal(c32, (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float32))
    assert np.array_equal(c16, oracle.f32_to_bf16_bits_np(c32))
    # normal data: within the sequential-fold bound of the exact product
    a = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (8, 300)).astype(np.float32))
    b = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (300, 40)).astype(np.float32))
    af, bf = oracle.bf16_bits_to_f32(a).astype(np.float64), oracle.bf16_bits_to_f32(b).astype(np.float64)
    c32, _ = oracle.matmul_bf16(a, b)
    bound = 300 * 2.0 ** -24 * (np.abs(af) @ np.abs(bf))
    assert np.all(np.abs(c32 - af @ bf) <= bound)
    # row subset returns the same rows
    rows = np.array([5, 0, 7], np.uint64)
    sub32, _ = oracle.matmul_bf16(a, b, rows=rows)
    assert np.array_equal(sub32, c32[[5, 0, 7]])


@pytest.mark.parametrize("n,m,k", [(1, 1, 1), (5, 3, 0), (7, 33, 129), (19, 64, 300),
                                   (3, 200, 4096)])
def test_bf16_gemm_is_f32_fold_on_widened_inputs(n, m, k):
    """or_matmul_bf16_seq is defined as the pinned f32 fold (or_matmul_f32_seq:
    k ascending from +0, separate * and +) on exactly widened inputs, then
    RNE to bf16: bitwise, on ragged shapes and with N(0,1) data whose partial
    sums round at almost every step (a wrong k order or a dropped term would
    change the bits)."""
    rng = np.random.default_rng(n * 7919 + m * 31 + k)
    a = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (n, k)).astype(np.float32))
    b = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (k, m)).astype(np.float32))
    c32, c16 = oracle.matmul_bf16(a, b)
    ref = oracle.matmul_f32(oracle.bf16_bits_to_f32(a), oracle.bf16_bits_to_f32(b))
    assert np.array_equal(c32.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(c16, oracle.f32_to_bf16_bits_np(ref))
    if k >= 2:  # the k order matters for these inputs: reversing it changes bits
        rev = oracle.matmul_f32(oracle.bf16_bits_to_f32(a)[:, ::-1].copy(),
                                oracle.bf16_bits_to_f32(b)[::-1].copy())
        assert not np.array_equal(rev.view(np.uint32), ref.view(np.uint32)) or k < 8


# ---------------------------------------------------------------- attention
def _rand_bf16(rng, shape, scale=1.0):
    return oracle.f32_to_bf16_bits_np((rng.normal(0, 1, shape) * scale).astype(np.float32))


def test_attention_composition_of_pinned_pieces():
    """s = q.K^T (the matmul fold over d), * scale, softmax, then p.V (the
    matmul fold over t): bitwise the composition of the pinned oracles."""
    rng = np.random.default_rng(5)
    B, H, L, D = 2, 3, 37, 128
    q, k, v = _rand_bf16(rng, (B, H, D)), _rand_bf16(rng, (B, H, L, D)), _rand_bf16(rng, (B, H, L, D))
    lens = np.array([37, 20], np.uint32)
    scale = 1.0 / math.sqrt(D)
    o = oracle.attn_decode(q, k, v, lens, scale)
    for b in range(B):
        for h in range(H):
            n = int(lens[b])
            qf = oracle.bf16_bits_to_f32(q[b, h]).reshape(1, D)
            kf = oracle.bf16_bits_to_f32(k[b, h, :n])
            vf = oracle.bf16_bits_to_f32(v[b, h, :n])
            s = oracle.matmul_f32(qf, np.ascontiguousarray(kf.T))[0]
            s = (s * np.float32(scale)).astype(np.float32)
            p = oracle.softmax_f32(s).reshape(1, n)
            ref = oracle.matmul_f32(p, vf)[0]
            assert np.array_equal(ref.view(np.uint32), o[b, h].view(np.uint32)), (b, h)


def test_attention_closed_forms():
    rng = np.random.default_rng(9)
    B, H, L, D = 1, 2, 16, 128
    q, k, v = _rand_bf16(rng, (B, H, D)), _rand_bf16(rng, (B, H, L, D)), _rand_bf16(rng, (B, H, L, D))
    # one position: p_0 = c0 / (0 + c0) = 1 exactly, so o = v_0 exactly
    o = oracle.attn_decode(q, k, v, np.array([1], np.uint32), 0.125)
    assert np.array_equal(o[0], oracle.bf16_bits_to_f32(v[0, :, 0]))
    # zero positions: every fold is empty, o = +0
    o = oracle.attn_decode(q, k, v, np.array([0], np.uint32), 0.125)
    assert np.all(o.view(np.uint32) == 0)
    # constant V: o_d = c * sum(p) ~ c
    vc = np.full((B, H, L, D), oracle.f32_to_bf16_bits_np(np.array([0.75], np.float32))[0], np.uint16)
    o = oracle.attn_decode(q, k, vc, np.array([16], np.uint32), 0.125)
    assert np.abs(o - 0.75).max() < 1e-5


def test_attention_vs_float64_softmax_attention():
    rng = np.random.default_rng(13)
    B, H, L, D = 2, 2, 300, 128
    q, k, v = _rand_bf16(rng, (B, H, D)), _rand_bf16(rng, (B, H, L, D)), _rand_bf16(rng, (B, H, L, D))
    lens = np.array([300, 129], np.uint32)
    scale = 1.0 / math.sqrt(D)
    o = oracle.attn_decode(q, k, v, lens, scale)
    for b in range(B):
        for h in range(H):
            n = int(lens[b])
            qf = oracle.bf16_bits_to_f32(q[b, h]).astype(np.float64)
            kf = oracle.bf16_bits_to_f32(k[b, h, :n]).astype(np.float64)
            vf = oracle.bf16_bits_to_f32(v[b, h, :n]).astype(np.float64)
            s = kf @ qf * scale
            p = np.exp(s - s.max())
            p /= p.sum()
            ref = p @ vf
            # exp~ is accurate to ~1.3% (relative), the rest to f32 rounding
            assert np.abs(o[b, h] - ref).max() < 0.03 * np.abs(vf).max(), (b, h)
