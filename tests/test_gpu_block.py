"""GPU parity of the decoder-block pieces: bitwise against the oracle.

Each kernel reproduces its stdlib op's node order (nn.rmsnorm's serial
square-sum fold and six-step Newton sqrt, nn.silu, math.sin-approx-full,
tensor.argmax-f32's NaN and tie behaviour), so outputs must match bit for
bit, including specials (zeros, NaN, inf, ties of +0/-0).  The causal
attention's queries must each equal the decode attention over their prefix.
"""
import math

import numpy as np
import pytest

import catena_amd as ca
import oracle
from oracle import decoder as od
from gpu_util import dev_normal_bf16, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _init():
    say("init device 0")
    ca.init(0)


def _bitwise(got, want):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape
    if got.dtype == np.float32:
        gn, wn = np.isnan(got), np.isnan(want)
        assert np.array_equal(gn, wn)
        got, want = got[~gn].view(np.uint32), want[~wn].view(np.uint32)
    assert np.array_equal(got, want), int(np.sum(got != want))


def _rows(rows, n, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((rows, n)) * scale).astype(np.float32)


@pytest.mark.parametrize("rows,n", [(1, 6), (3, 2048), (2, 4097), (5, 5632), (1, 1), (4, 12),
                                    (2, 31), (2, 33), (3, 2049), (1, 6143), (1, 20000),
                                    (2, 1023), (2, 1024), (2, 1030)])
def test_rmsnorm_f32(rows, n):
    say(f"rmsnorm rows={rows} n={n}")
    x = _rows(rows, n, rows * 31 + n, scale=3.0)
    if n == 6:
        x[0] = [1.0, 2.0, 4.0, -1.0, -9.0, 13.29]  # catena-lang/tests/runtime.rs:1011-1044
    xb, yb = ca.Buffer.from_array(x), ca.Buffer(x.nbytes)
    ca.rmsnorm_f32(xb, yb, rows, n)
    _bitwise(yb.read(np.float32, (rows, n)), oracle.rmsnorm_f32(x))


def test_rmsnorm_row_limit():
    """The row and its squares sit in LDS beside the kernel's static f32:
    16 + 8 n <= 163,840 B, so 20,476 elements run and 20,480 are refused
    with CATENA_ERR_UNSUPPORTED before any launch."""
    x = _rows(1, 20480, 3)
    xb, yb = ca.Buffer.from_array(x), ca.Buffer(x.nbytes)
    say("rmsnorm n=20480 (refused)")
    with pytest.raises(ca.CatenaError) as e:
        ca.rmsnorm_f32(xb, yb, 1, 20480)
    assert e.value.status == 2
    say("rmsnorm n=20476")
    ca.rmsnorm_f32(xb, yb, 1, 20476)
    _bitwise(yb.read(np.float32, (1, 20480))[:, :20476], oracle.rmsnorm_f32(x[:, :20476]))


@pytest.mark.parametrize("n", [64, 2048])
def test_rmsnorm_specials(n):
    x = _rows(6, n, 5)
    x[0] = 0.0                      # sum 0: rms = sqrt(eps)
    x[1, 3] = np.nan                # NaN propagates through the fold
    x[2, 7] = np.inf
    x[3] = 3e19                     # squares overflow to inf
    x[4] = 1e-30                    # squares underflow (subnormal/zero)
    x[5, ::2] = -0.0
    xb, yb = ca.Buffer.from_array(x), ca.Buffer(x.nbytes)
    say(f"rmsnorm specials n={n}")
    ca.rmsnorm_f32(xb, yb, 6, n)
    _bitwise(yb.read(np.float32, (6, n)), oracle.rmsnorm_f32(x))


@pytest.mark.parametrize("n", [2048, 12, 5632, 1028, 8, 2044])
def test_rmsnorm_many_rows(n):
    """2,100 rows (more than one round of workgroups on the device): bitwise
    the oracle on normal and special rows (zero, NaN, inf, overflowing and
    underflowing squares, -0), and bitwise the same rows computed as a small
    batch."""
    rows = 2100
    x = _rows(rows, n, n + 17, scale=2.0)
    x[0] = 0.0
    x[1, 3] = np.nan
    x[2, 7] = np.inf
    x[3] = 3e19
    x[4] = 1e-30
    x[5, ::2] = -0.0
    xb, yb = ca.Buffer.from_array(x), ca.Buffer(x.nbytes)
    say(f"rmsnorm {rows} rows n={n}")
    ca.rmsnorm_f32(xb, yb, rows, n)
    got = yb.read(np.float32, (rows, n))
    _bitwise(got, oracle.rmsnorm_f32(x))
    few = ca.Buffer.from_array(np.ascontiguousarray(x[:9]))
    yf = ca.Buffer(9 * n * 4)
    ca.rmsnorm_f32(few, yf, 9, n)
    assert np.array_equal(yf.read(np.uint32, (9, n)), got[:9].view(np.uint32))


@pytest.mark.parametrize("rows", [3000, 2049])
def test_residual_rmsnorm_many_rows(rows):
    """The residual add, h output and bf16 output over many rows, then the
    same with a row index selecting 100 fewer rows: both bitwise the
    oracle."""
    n = 2048
    x = _rows(rows, n, 71)
    r = _rows(rows, n, 72, scale=0.5)
    x[5, 9] = np.nan
    r[6] = 3e19
    xb, rb = ca.Buffer.from_array(x), ca.Buffer.from_array(r)
    hb, yb = ca.Buffer(rows * n * 4), ca.Buffer(rows * n * 2)
    say(f"residual rmsnorm {rows} rows")
    ca.residual_rmsnorm_bf16(xb, rb, None, hb, yb, rows, n)
    h, y = od.residual_rmsnorm_bf16(x, r)
    _bitwise(hb.read(np.float32, (rows, n)), h)
    _bitwise(yb.read(np.uint16, (rows, n)), y)
    rows_out = rows - 100
    idx = np.random.default_rng(73).permutation(rows)[:rows_out].astype(np.uint32)
    ib = ca.Buffer.from_array(idx)
    say(f"residual rmsnorm {rows_out} indexed rows")
    ca.residual_rmsnorm_bf16(xb, rb, ib, hb, yb, rows_out, n)
    h, y = od.residual_rmsnorm_bf16(x[idx.astype(np.int64)], r[idx.astype(np.int64)])
    _bitwise(hb.read(np.float32, (rows_out, n)), h)
    _bitwise(yb.read(np.uint16, (rows_out, n)), y)


@pytest.mark.parametrize("use_resid,use_index,n", [(True, False, 2048), (False, False, 256),
                                                   (True, True, 2048), (True, True, 10)])
def test_residual_rmsnorm_bf16(use_resid, use_index, n):
    rows_in = 9
    x = _rows(rows_in, n, n + 1)
    r = _rows(rows_in, n, n + 2, scale=0.5)
    idx = np.array([8, 0, 3], np.uint32) if use_index else None
    rows_out = 3 if use_index else rows_in
    xb, rb = ca.Buffer.from_array(x), ca.Buffer.from_array(r)
    ib = ca.Buffer.from_array(idx) if use_index else None
    hb, yb = ca.Buffer(rows_out * n * 4), ca.Buffer(rows_out * n * 2)
    say(f"residual rmsnorm resid={use_resid} index={use_index} n={n}")
    ca.residual_rmsnorm_bf16(xb, rb if use_resid else None, ib, hb, yb, rows_out, n)
    src = idx.astype(np.int64) if use_index else np.arange(rows_in)
    h, y = od.residual_rmsnorm_bf16(x[src], r[src] if use_resid else None)
    _bitwise(hb.read(np.float32, (rows_out, n)), h)
    _bitwise(yb.read(np.uint16, (rows_out, n)), y)


def test_embed():
    V, d = 40, 256
    table = dev_normal_bf16(V * d, 7, 0)
    tok = np.array([0, 39, 5, 5, 40, 1000000], np.uint32)  # last two out of range
    tb = ca.Buffer.from_array(tok)
    x = ca.Buffer(tok.size * d * 4)
    say("embed")
    ca.embed_bf16(tb, table, x, tok.size, V, d)
    got = x.read(np.float32, (tok.size, d))
    t = table.read(np.uint16, (V, d))
    _bitwise(got[:4], oracle.bf16_bits_to_f32(t[tok[:4].astype(np.int64)]))
    assert np.all(np.isnan(got[4:]))


def test_rope_inv_freq_matches_oracle():
    for D, base in [(128, 10000.0), (64, 500000.0)]:
        assert np.array_equal(ca.rope_inv_freq(D, base).view(np.uint32),
                              oracle.rope_inv_freq(D, base).view(np.uint32))


@pytest.mark.parametrize("B,Tq,H,L,lens", [(2, 3, 2, 8, [5, 3]), (3, 1, 4, 640, [640, 1, 77]),
                                           (2, 16, 3, 600, [600, 16])])
def test_rope_qkv_store(B, Tq, H, L, lens):
    D = 128
    R = B * Tq
    rng = np.random.default_rng(B * 100 + Tq)
    qkv = (rng.standard_normal((R, 3 * H * D)) * 2).astype(np.float32)
    inv = ca.rope_inv_freq(D, 10000.0)
    kc = ca.Buffer(B * H * L * D * 2)
    vc = ca.Buffer(B * H * L * D * 2)
    sentinel = np.full(B * H * L * D, 0xABCD, np.uint16)
    kc.write(sentinel)
    vc.write(sentinel)
    qb = ca.Buffer(R * H * D * 2)
    say(f"rope qkv B={B} Tq={Tq} H={H} L={L} lens={lens}")
    ca.rope_qkv_bf16(ca.Buffer.from_array(qkv), ca.Buffer.from_array(inv),
                     ca.Buffer.from_array(np.array(lens, np.uint32)), qb, kc, vc, B, Tq, H, D, L)
    q, k, v, pos = od.rope_qkv(qkv, inv, lens, B, Tq, H, D)
    _bitwise(qb.read(np.uint16, (R, H * D)), q)
    kg = kc.read(np.uint16, (B, H, L, D))
    vg = vc.read(np.uint16, (B, H, L, D))
    written = np.zeros((B, L), bool)
    for r in range(R):
        b = r // Tq
        _bitwise(kg[b, :, pos[r]], k[r])
        _bitwise(vg[b, :, pos[r]], v[r])
        written[b, pos[r]] = True
    untouched = ~written
    assert np.all(kg.transpose(0, 2, 1, 3)[untouched] == 0xABCD)
    assert np.all(vg.transpose(0, 2, 1, 3)[untouched] == 0xABCD)


def test_rope_large_positions_against_libm():
    """Rotation at position 4095 stays within 2e-4 (plus bf16 rounding) of the
    libm value, so both the range reduction and the quadrant map hold."""
    D, H, B, L = 128, 1, 1, 4096
    lens = [4096]
    qkv = np.random.default_rng(3).standard_normal((1, 3 * D)).astype(np.float32)
    inv = ca.rope_inv_freq(D, 10000.0)
    qb = ca.Buffer(D * 2)
    kc, vc = ca.Buffer(B * H * L * D * 2), ca.Buffer(B * H * L * D * 2)
    say("rope at position 4095")
    ca.rope_qkv_bf16(ca.Buffer.from_array(qkv), ca.Buffer.from_array(inv),
                     ca.Buffer.from_array(np.array(lens, np.uint32)), qb, kc, vc, 1, 1, H, D, L)
    q = oracle.bf16_bits_to_f32(qb.read(np.uint16)).astype(np.float64)
    th = 4095.0 * inv.astype(np.float64)
    x1, x2 = qkv[0, :64].astype(np.float64), qkv[0, 64:128].astype(np.float64)
    want = np.concatenate([x1 * np.cos(th) - x2 * np.sin(th), x2 * np.cos(th) + x1 * np.sin(th)])
    assert np.abs(q - want).max() < 2e-4 + 2 ** -7 * np.abs(want).max()


@pytest.mark.parametrize("rows,F,group", [(3, 1024, 0), (8, 5632, 0), (1, 4, 0), (8, 5632, 64),
                                           (2, 256, 4)])
def test_silu_mul(rows, F, group):
    rng = np.random.default_rng(F + group)
    gu = (rng.standard_normal((rows, 2 * F)) * 4).astype(np.float32)
    gu[0, :4] = [0.0, -0.0, 100.0, -100.0]
    out = ca.Buffer(rows * F * 2)
    say(f"silu_mul rows={rows} F={F} group={group}")
    ca.silu_mul_bf16(ca.Buffer.from_array(gu), out, rows, F, group)
    _bitwise(out.read(np.uint16, (rows, F)), od.silu_mul_bf16(gu, F, group))


def _argmax_rows(rows):
    n = max(len(r) for r in rows)
    assert all(len(r) == n for r in rows)
    x = np.array(rows, np.float32)
    idx = ca.Buffer(len(rows) * 4)
    ca.argmax_f32(ca.Buffer.from_array(x), idx, len(rows), n)
    return idx.read(np.uint32)


def test_argmax_special_rows():
    nan, inf = np.nan, np.inf
    rows = [
        [1.0, 3.0, 3.0, 2.0, 0.0],
        [nan, 1.0, 5.0, 5.0, 2.0],
        [1.0, 9.0, nan, 0.5, 0.7],
        [1.0, 2.0, 3.0, 4.0, nan],
        [-inf, -inf, -inf, -inf, -inf],
        [-0.0, 0.0, -0.0, 0.0, -1.0],
        [0.0, -0.0, 0.0, -0.0, -1.0],
        [nan, nan, nan, nan, nan],
        [inf, 1.0, inf, nan, -inf],
    ]
    say("argmax special rows")
    got = _argmax_rows(rows)
    want = [oracle.argmax_f32(np.array(r, np.float32)) for r in rows]
    assert list(got) == want


def test_argmax_golden_and_large():
    import json
    import os
    g = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                    "reference_known_answers.json")))
    for values, expect in g["argmax_first_index"]["cases"]:
        say(f"argmax golden {values}")
        assert int(_argmax_rows([values])[0]) == expect
    rng = np.random.default_rng(11)
    x = rng.standard_normal((8, 32000)).astype(np.float32)
    x[3, 17] = x[3, 29999] = 50.0  # tie: first wins
    x[5, 100] = np.nan
    idx = ca.Buffer(8 * 4)
    say("argmax 8 x 32000")
    ca.argmax_f32(ca.Buffer.from_array(x), idx, 8, 32000)
    assert list(idx.read(np.uint32)) == [oracle.argmax_f32(r) for r in x]


def _attn_inputs(B, Tq, H, L, seed):
    D = 128
    q = dev_normal_bf16(B * Tq * H * D, seed, 0)
    k = dev_normal_bf16(B * H * L * D, seed, 1)
    v = dev_normal_bf16(B * H * L * D, seed, 2)
    return q, k, v


@pytest.mark.parametrize("B,Tq,H,L,lens", [(2, 4, 3, 64, [10, 4]), (1, 7, 2, 300, [300]),
                                           (2, 64, 4, 512, [512, 100]), (3, 2, 1, 16, [1, 0, 16])])
def test_attention_causal_matches_prefix_decode(B, Tq, H, L, lens):
    D = 128
    q, k, v = _attn_inputs(B, Tq, H, L, B * 10 + Tq)
    lb = ca.Buffer.from_array(np.array(lens, np.uint32))
    scale = 1.0 / math.sqrt(D)
    o32 = ca.Buffer(B * Tq * H * D * 4)
    o16 = ca.Buffer(B * Tq * H * D * 2)
    say(f"causal attention B={B} Tq={Tq} H={H} L={L} lens={lens}")
    ca.attn_causal_bf16(q, k, v, lb, o32, B, Tq, H, L, D, scale, out_f32=True)
    ca.attn_causal_bf16(q, k, v, lb, o16, B, Tq, H, L, D, scale, out_f32=False)
    want = od.attn_causal(q.read(np.uint16), k.read(np.uint16, (B, H, L, D)),
                          v.read(np.uint16, (B, H, L, D)), lens, B, Tq, H, D, scale)
    g32 = o32.read(np.float32, (B * Tq, H * D))
    _bitwise(g32, want)
    _bitwise(o16.read(np.uint16, (B * Tq, H * D)), oracle.f32_to_bf16_bits_np(want))


def test_attention_causal_random_configs():
    """Ten seeded random causal configurations (Tq from 2 to 80, so both the
    16-query prefill kernel and the one-query kernel run; cached prefixes
    with lens > Tq, sequences shorter than Tq, empty ones; random scales):
    f32 output bitwise the oracle's causal attention, bf16 output its RNE."""
    D = 128
    rng = np.random.default_rng(31337)
    for i in range(10):
        B, H = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        Tq = int(rng.integers(2, 81))
        L = int(rng.integers(Tq, 700))
        lens = [int(x) for x in rng.integers(0, L + 1, B)]
        if i % 3 == 0:
            lens[0] = L
        scale = float(np.float32(rng.uniform(0.05, 0.2)))
        q, k, v = _attn_inputs(B, Tq, H, L, 900 + i)
        lb = ca.Buffer.from_array(np.array(lens, np.uint32))
        o32 = ca.Buffer(B * Tq * H * D * 4)
        o16 = ca.Buffer(B * Tq * H * D * 2)
        say(f"causal attention random config B={B} Tq={Tq} H={H} L={L} lens={lens} scale={scale}")
        ca.attn_causal_bf16(q, k, v, lb, o32, B, Tq, H, L, D, scale, out_f32=True)
        ca.attn_causal_bf16(q, k, v, lb, o16, B, Tq, H, L, D, scale, out_f32=False)
        want = od.attn_causal(q.read(np.uint16), k.read(np.uint16, (B, H, L, D)),
                              v.read(np.uint16, (B, H, L, D)), lens, B, Tq, H, D, scale)
        _bitwise(o32.read(np.float32, (B * Tq, H * D)), want)
        _bitwise(o16.read(np.uint16, (B * Tq, H * D)), oracle.f32_to_bf16_bits_np(want))


def test_attention_causal_prefill_nan_inf_tie_scores():
    """The 16-query prefill kernel (Tq >= 8) on scores with a NaN inside the
    prefix (the max restarts after it), a NaN at exactly one query's last
    position (that query's max is the NaN), an overflowing score, all-equal
    (+0) scores, and a partial last block of queries (Tq = 20)."""
    B, Tq, H, L, D = 2, 20, 4, 48, 128
    lens = [48, 30]
    rng = np.random.default_rng(21)
    q16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B * Tq * H * D,)).astype(np.float32))
    k32 = rng.normal(0, 1, (B, H, L, D)).astype(np.float32)
    k32[0, 0, 10, 5] = np.nan      # positions 11.. of every query of b 0 follow a NaN
    k32[0, 1, 35, 0] = np.nan      # b 0, query 6 has 36 positions: its last one is NaN
    k32[0, 2, 3, :] = 1e30         # overflowing score
    k32[0, 3, :, :] = 0.0          # every score +0
    k16 = oracle.f32_to_bf16_bits_np(k32)
    v16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B, H, L, D)).astype(np.float32))
    q, k, v = ca.Buffer.from_array(q16), ca.Buffer.from_array(k16), ca.Buffer.from_array(v16)
    lb = ca.Buffer.from_array(np.array(lens, np.uint32))
    scale = 1.0 / math.sqrt(D)
    o32 = ca.Buffer(B * Tq * H * D * 4)
    say("causal prefill attention NaN / inf / tie scores")
    ca.attn_causal_bf16(q, k, v, lb, o32, B, Tq, H, L, D, scale, out_f32=True)
    want = od.attn_causal(q16, k16, v16, lens, B, Tq, H, D, scale)
    _bitwise(o32.read(np.float32, (B * Tq, H * D)), want)


def test_attention_prefill_mfma_fold_range_guard():
    """The prefill kernel folds q.k on the matrix cores (one rounding per
    step, exact products) only while every nonzero q / k magnitude is in
    [2^-63, 2^63); otherwise the workgroup refolds with v_mul_f32 +
    v_add_f32.  Heads scaled so that products fall in the denormal range
    (head 1: fused and separately rounded steps differ there) or overflow
    (head 2), beside heads inside the range (0, 3) and at its edges (4:
    2^-63 and just below 2^63): all bitwise the oracle."""
    B, Tq, H, L, D = 2, 40, 5, 64, 128
    lens = [64, 40]
    rng = np.random.default_rng(33)
    q32 = rng.normal(0, 1, (B, Tq, H, D)).astype(np.float32)
    k32 = rng.normal(0, 1, (B, H, L, D)).astype(np.float32)
    q32[:, :, 1] *= 2.0 ** -68
    k32[:, 1] *= 2.0 ** -68
    q32[:, :, 2] *= 2.0 ** 66
    k32[:, 2] *= 2.0 ** 64
    q32[:, :, 3] *= 2.0 ** -30
    k32[:, 3] *= 2.0 ** 30
    edge = np.where(rng.random((B, H, L, D)) < 0.5, 2.0 ** -63, np.float32(1.99) * 2.0 ** 62)
    k32[:, 4] = (np.sign(k32[:, 4]) * edge[:, 4]).astype(np.float32)
    q16 = oracle.f32_to_bf16_bits_np(q32).reshape(-1)
    k16 = oracle.f32_to_bf16_bits_np(k32)
    v16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B, H, L, D)).astype(np.float32))
    q, k, v = ca.Buffer.from_array(q16), ca.Buffer.from_array(k16), ca.Buffer.from_array(v16)
    lb = ca.Buffer.from_array(np.array(lens, np.uint32))
    scale = 1.0 / math.sqrt(D)
    o32 = ca.Buffer(B * Tq * H * D * 4)
    say("prefill attention: MFMA fold range guard (denormal / overflow / edge heads)")
    ca.attn_causal_bf16(q, k, v, lb, o32, B, Tq, H, L, D, scale, out_f32=True)
    want = od.attn_causal(q16, k16, v16, lens, B, Tq, H, D, scale)
    _bitwise(o32.read(np.float32, (B * Tq, H * D)), want)


def test_attention_prefill_pv_products_specials():
    """The prefill kernel forms the P·V products on the matrix cores with a
    zero accumulator (fl(p * v), then the adds on the VALU).  Heads that
    push those products to the edges: head 0 spreads the scores over
    hundreds (exp~ of the shifted scores, wrapped powers of two included,
    gives tiny and denormal p); head 1 puts NaN, +-inf, +-0, bf16 denormals
    and the largest bf16 values into V at random positions; head 2 pairs
    tiny p with denormal V (products underflow to denormals or zero); head
    3 plain.  L = 100 (not a multiple of the 64-key blocks), Tq = 40 (a
    partial last query block), and a sequence shorter than Tq.  f32 output
    bitwise the oracle (NaN positions equal)."""
    B, Tq, H, L, D = 3, 40, 4, 100, 128
    lens = [100, 60, 25]
    rng = np.random.default_rng(707)
    q32 = rng.normal(0, 1, (B, Tq, H, D)).astype(np.float32)
    k32 = rng.normal(0, 1, (B, H, L, D)).astype(np.float32)
    v32 = rng.normal(0, 1, (B, H, L, D)).astype(np.float32)
    q32[:, :, 0] *= 16.0
    k32[:, 0] *= 4.0
    q32[:, :, 2] *= 12.0
    k32[:, 2] *= 4.0
    v16 = oracle.f32_to_bf16_bits_np(v32)
    specials = np.array([0x7FC0, 0xFFC1, 0x7F80, 0xFF80, 0x0000, 0x8000, 0x0001, 0x807F,
                         0x0040, 0x7F7F, 0xFF7F], np.uint16)
    msk = rng.random((B, L, D)) < 0.02
    v16[:, 1][msk] = rng.choice(specials, int(msk.sum()))
    v16[:, 2] = (rng.integers(1, 0x80, (B, L, D)) | (rng.integers(0, 2, (B, L, D)) << 15)).astype(np.uint16)
    q16 = oracle.f32_to_bf16_bits_np(q32).reshape(-1)
    k16 = oracle.f32_to_bf16_bits_np(k32)
    q, k, v = ca.Buffer.from_array(q16), ca.Buffer.from_array(k16), ca.Buffer.from_array(v16)
    lb = ca.Buffer.from_array(np.array(lens, np.uint32))
    scale = 1.0 / math.sqrt(D)
    o32 = ca.Buffer(B * Tq * H * D * 4)
    say("prefill attention: P.V products at the edges (tiny p, V specials, denormal V)")
    ca.attn_causal_bf16(q, k, v, lb, o32, B, Tq, H, L, D, scale, out_f32=True)
    want = od.attn_causal(q16, k16, v16, lens, B, Tq, H, D, scale)
    got = o32.read(np.float32, (B * Tq, H * D))
    _bitwise(got, want)
    # the heads reach the cases they are for
    w = want.reshape(B, Tq, H, D)
    assert np.isnan(w[:, :, 1]).any() and np.isinf(w[:, :, 1]).any()
    tiny = np.abs(w[:, :, 2])
    assert ((tiny > 0) & (tiny < np.float32(2.0 ** -126))).any()


def test_attention_causal_tq1_equals_decode_kernel():
    B, H, L, D = 4, 8, 1024, 128
    q, k, v = _attn_inputs(B, 1, H, L, 99)
    lb = ca.Buffer.from_array(np.array([1024, 3, 700, 64], np.uint32))
    a, b = ca.Buffer(B * H * D * 4), ca.Buffer(B * H * D * 4)
    say("causal Tq=1 vs decode kernel")
    ca.attn_causal_bf16(q, k, v, lb, a, B, 1, H, L, D, 1 / math.sqrt(D), out_f32=True)
    ca.attn_decode_bf16(q, k, v, lb, b, B, H, L, D, 1 / math.sqrt(D))
    assert np.array_equal(a.read(np.uint32), b.read(np.uint32))


def test_programs_rmsnorm_and_argmax():
    rt = ca.Runtime([])
    x = [1.0, 2.0, 4.0, -1.0, -9.0, 13.29]  # catena-lang/tests/runtime.rs:1011-1044
    say("runtime exec nn.rmsnorm")
    [res] = rt.exec("nn.rmsnorm", [rt.mem_f32(x)], 1)
    got = ca.mem_to_array(res.get(), np.float32)
    _bitwise(got, oracle.rmsnorm_f32(np.array(x, np.float32)))
    ms = sum(v * v for v in x) / len(x)
    assert np.abs(got - np.array(x) / math.sqrt(ms + 1e-5)).max() < 3e-3
    ca.mem_free(res.get())
    say("runtime exec tensor.argmax-f32")
    [res] = rt.exec("tensor.argmax-f32", [rt.mem_f32([1.0, 3.0, 3.0, 2.0])], 1)
    assert res.get() == 1  # first index of the tie (catena-lang/tests/runtime.rs:1176-1197)


def test_argmax_chunked_nan_and_tie_patterns():
    """Rows long enough to span several workgroups (4096 elements each):
    NaNs and ties placed on and across chunk boundaries."""
    n = 3 * 4096 + 17
    rng = np.random.default_rng(21)
    x = rng.standard_normal((7, n)).astype(np.float32)
    x[0, 4095] = np.nan                      # NaN at a chunk's last element
    x[1, 4096] = np.nan                      # ... at a chunk's first element
    x[1, 100] = 99.0                         # maximum before the NaN is ignored
    x[2, n - 1] = np.nan                     # final NaN is the answer
    x[3, [10, 5000, 9000]] = 77.0            # tie across chunks: first wins
    x[4, 8192:] = np.nan                     # NaN run to the end
    x[5, 3] = np.nan
    x[5, 12000] = np.nan
    x[5, [12001, 12100]] = 40.0              # tie after the last NaN
    x[6, :] = -np.inf
    idx = ca.Buffer(7 * 4)
    say("argmax chunked patterns")
    ca.argmax_f32(ca.Buffer.from_array(x), idx, 7, n)
    assert list(idx.read(np.uint32)) == [oracle.argmax_f32(r) for r in x]
    # the same rows again: the completion counters were returned to zero
    ca.argmax_f32(ca.Buffer.from_array(x), idx, 7, n)
    assert list(idx.read(np.uint32)) == [oracle.argmax_f32(r) for r in x]


@pytest.mark.parametrize("B,Tq,H,L,lens", [(2, 37, 3, 200, [200, 37]), (1, 512, 2, 640, [512]),
                                           (3, 8, 2, 96, [96, 8, 30]), (2, 100, 1, 700, [700, 120]),
                                           (1, 12, 2, 1000, [1000]), (1, 20, 2, 1200, [1200])])
def test_attention_prefill_kernel_equals_per_query_kernel(B, Tq, H, L, lens):
    """The causal attention (the 16-query-block kernel for Tq >= 8 while its
    score buffer fits, L <= 1,088; the one-query kernel beyond, as in the
    last case) against the decode kernel run once per query on that query's
    prefix (same bits by construction), including cached prefixes
    (lens > Tq), partial last blocks and sequences shorter than Tq."""
    D = 128
    q, k, v = _attn_inputs(B, Tq, H, L, B * 7 + Tq)
    lb = ca.Buffer.from_array(np.array(lens, np.uint32))
    scale = 1.0 / math.sqrt(D)
    a32 = ca.Buffer(B * Tq * H * D * 4)
    a16 = ca.Buffer(B * Tq * H * D * 2)
    say(f"prefill attention B={B} Tq={Tq} H={H} L={L} lens={lens}")
    ca.attn_causal_bf16(q, k, v, lb, a32, B, Tq, H, L, D, scale, out_f32=True)
    ca.attn_causal_bf16(q, k, v, lb, a16, B, Tq, H, L, D, scale, out_f32=False)
    got = a32.read(np.float32, (B, Tq, H, D))
    assert np.array_equal(a16.read(np.uint16, (B, Tq, H, D)),
                          oracle.f32_to_bf16_bits_np(got))
    q_host = q.read(np.uint16, (B, Tq, H, D))
    ob = ca.Buffer(B * H * D * 4)
    for t in range(Tq):
        qt = ca.Buffer.from_array(np.ascontiguousarray(q_host[:, t]))
        ln = ca.Buffer.from_array(np.maximum(np.array(lens, np.int64) - (Tq - 1 - t), 0)
                                  .astype(np.uint32))
        ca.attn_decode_bf16(qt, k, v, ln, ob, B, H, L, D, scale)
        assert np.array_equal(got[:, t].view(np.uint32), ob.read(np.uint32, (B, H, D))), t
    if B * Tq * H <= 4096:
        want = od.attn_causal(q.read(np.uint16), k.read(np.uint16, (B, H, L, D)),
                              v.read(np.uint16, (B, H, L, D)), lens, B, Tq, H, D, scale)
        _bitwise(a32.read(np.float32, (B * Tq, H * D)), want)
