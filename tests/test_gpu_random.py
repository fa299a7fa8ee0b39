"""Seeded random configurations of the row kernels and fused epilogues.

The parametrized tests elsewhere pin chosen shapes and special values; these
draw shapes, lengths, groupings and special-value positions at random (fixed
seeds, so a failure names its case and repeats) and hold every output to the
same bar: bitwise the oracle for the elementwise and fold kernels, bitwise
the unfused GPU pair for the fused GEMM epilogues.
"""
import numpy as np
import pytest

import catena_amd as ca
import oracle
from oracle import decoder as od
from gpu_util import dev_normal_bf16, say

pytestmark = pytest.mark.gpu

SPECIALS = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3e38, -3e38, 1e-40, -1e-40, 1e-30],
                    np.float32)


@pytest.fixture(scope="module", autouse=True)
def _init():
    say("init device 0")
    ca.init(0)


def _bits_nan_aware(got, want):
    """Bitwise equality, NaN for NaN: a NaN's sign and payload are not part
    of the result (the host's default NaN is negative, the GPU's positive).
    uint16 arrays are bf16 bit patterns."""
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    if got.dtype == np.float32:
        gn, wn = np.isnan(got), np.isnan(want)
        got, want = got[~gn].view(np.uint32), want[~wn].view(np.uint32)
    elif got.dtype == np.uint16:
        gn, wn = (got & 0x7FFF) > 0x7F80, (want & 0x7FFF) > 0x7F80
        got, want = got[~gn], want[~wn]
    else:
        gn = wn = np.zeros(got.shape, bool)
    assert np.array_equal(gn, wn), int(np.sum(gn != wn))
    assert np.array_equal(got, want), int(np.sum(got != want))


def _rows(rng, rows, n, specials_frac):
    x = (rng.standard_normal((rows, n)) * np.exp(rng.uniform(-3, 3, (rows, 1)))).astype(np.float32)
    if specials_frac:
        m = rng.random((rows, n)) < specials_frac
        x[m] = rng.choice(SPECIALS, int(m.sum()))
    return x


def test_softmax_random_rows():
    rng = np.random.default_rng(71)
    for i in range(12):
        rows, n = int(rng.integers(1, 6)), int(rng.integers(1, 6000))
        x = _rows(rng, rows, n, 0.002 if i % 2 else 0.0)
        say(f"softmax random rows={rows} n={n}")
        y = ca.Buffer(x.nbytes)
        ca.softmax_f32(ca.Buffer.from_array(x), y, rows, n)
        got = y.read(np.float32, (rows, n))
        for r in range(rows):
            _bits_nan_aware(got[r], oracle.softmax_f32(x[r]))


def test_folds_random_rows():
    rng = np.random.default_rng(72)
    for i in range(12):
        rows, n = int(rng.integers(1, 8)), int(rng.integers(1, 70000))
        x = _rows(rng, rows, n, 0.0005 if i % 3 == 0 else 0.0)
        xb, o = ca.Buffer.from_array(x), ca.Buffer(rows * 4)
        say(f"sum / mean / max random rows={rows} n={n}")
        ca.sum_f32(xb, o, rows, n)
        _bits_nan_aware(o.read(np.float32), np.array([oracle.fold_sum_f32(r) for r in x], np.float32))
        ca.mean_f32(xb, o, rows, n)
        want = np.array([np.float32(oracle.fold_sum_f32(r)) / np.float32(n) for r in x], np.float32)
        _bits_nan_aware(o.read(np.float32), want)
        ca.max_f32(xb, o, rows, n)
        _bits_nan_aware(o.read(np.float32), np.array([oracle.fold_max_f32(r) for r in x], np.float32))


def test_argmax_random_rows():
    """Random widths, values drawn from a small set so ties are common, and
    NaNs at random positions (the last NaN restarts the first-maximum fold)."""
    rng = np.random.default_rng(73)
    for i in range(12):
        rows, n = int(rng.integers(1, 10)), int(rng.integers(1, 70000))
        x = rng.integers(-20, 20, (rows, n)).astype(np.float32)
        if i % 2:
            m = rng.random((rows, n)) < 0.0005
            x[m] = np.nan
        if i % 3 == 0:
            x[0] = -np.inf
        idx = ca.Buffer(rows * 4)
        say(f"argmax random rows={rows} n={n}")
        ca.argmax_f32(ca.Buffer.from_array(x), idx, rows, n)
        assert list(idx.read(np.uint32)) == [oracle.argmax_f32(r) for r in x]


def test_rmsnorm_random_rows():
    rng = np.random.default_rng(74)
    for i in range(10):
        rows, n = int(rng.integers(1, 40)), int(rng.integers(1, 8000))
        x = _rows(rng, rows, n, 0.001 if i % 2 else 0.0)
        say(f"rmsnorm random rows={rows} n={n}")
        y = ca.Buffer(x.nbytes)
        ca.rmsnorm_f32(ca.Buffer.from_array(x), y, rows, n)
        _bits_nan_aware(y.read(np.float32, (rows, n)), oracle.rmsnorm_f32(x))


def test_residual_rmsnorm_random_rows():
    rng = np.random.default_rng(75)
    for i in range(10):
        rows_in, n = int(rng.integers(1, 300)), 4 * int(rng.integers(1, 1500))
        x = _rows(rng, rows_in, n, 0.0005 if i % 2 else 0.0)
        r = _rows(rng, rows_in, n, 0.0)
        use_index = i % 3 == 1
        use_resid = i % 4 != 3
        idx = rng.integers(0, rows_in, int(rng.integers(1, rows_in + 1))).astype(np.uint32) if use_index else None
        rows_out = idx.size if use_index else rows_in
        hb, yb = ca.Buffer(rows_out * n * 4), ca.Buffer(rows_out * n * 2)
        say(f"residual rmsnorm random rows={rows_out} n={n} resid={use_resid} index={use_index}")
        ca.residual_rmsnorm_bf16(ca.Buffer.from_array(x), ca.Buffer.from_array(r) if use_resid else None,
                                 ca.Buffer.from_array(idx) if use_index else None, hb, yb, rows_out, n)
        src = idx.astype(np.int64) if use_index else np.arange(rows_in)
        h, y = od.residual_rmsnorm_bf16(x[src], r[src] if use_resid else None)
        _bits_nan_aware(hb.read(np.float32, (rows_out, n)), h)
        _bits_nan_aware(yb.read(np.uint16, (rows_out, n)), y)


def test_silu_mul_random():
    rng = np.random.default_rng(76)
    for i in range(10):
        group = int(rng.choice([0, 4, 8, 64]))
        F = 4 * int(rng.integers(1, 2000))
        if group:
            F = group * max(1, F // group)
        rows = int(rng.integers(1, 20))
        gu = (rng.standard_normal((rows, 2 * F)) * 6).astype(np.float32)
        if i % 2:
            m = rng.random((rows, 2 * F)) < 0.002
            gu[m] = rng.choice(SPECIALS, int(m.sum()))
        out = ca.Buffer(rows * F * 2)
        say(f"silu_mul random rows={rows} F={F} group={group}")
        ca.silu_mul_bf16(ca.Buffer.from_array(gu), out, rows, F, group)
        _bits_nan_aware(out.read(np.uint16, (rows, F)), od.silu_mul_bf16(gu, F, group))


def test_rope_qkv_random():
    D = 128
    rng = np.random.default_rng(77)
    for i in range(8):
        B, Tq, H = int(rng.integers(1, 5)), int(rng.integers(1, 40)), int(rng.integers(1, 4))
        L = int(rng.integers(1, 700))
        lens = [int(x) for x in rng.integers(0, L + Tq + 3, B)]  # some past L, some shorter than Tq
        R = B * Tq
        qkv = (rng.standard_normal((R, 3 * H * D)) * 3).astype(np.float32)
        inv = ca.rope_inv_freq(D, float(rng.choice([10000.0, 500000.0])))
        kc, vc = ca.Buffer(B * H * L * D * 2), ca.Buffer(B * H * L * D * 2)
        sentinel = np.full(B * H * L * D, 0xABCD, np.uint16)
        kc.write(sentinel)
        vc.write(sentinel)
        qb = ca.Buffer(R * H * D * 2)
        say(f"rope qkv random B={B} Tq={Tq} H={H} L={L} lens={lens}")
        ca.rope_qkv_bf16(ca.Buffer.from_array(qkv), ca.Buffer.from_array(inv),
                         ca.Buffer.from_array(np.array(lens, np.uint32)), qb, kc, vc, B, Tq, H, D, L)
        q, k, v, pos = od.rope_qkv(qkv, inv, lens, B, Tq, H, D, max_len=L)
        _bits_nan_aware(qb.read(np.uint16, (R, H * D)), q)
        kg, vg = kc.read(np.uint16, (B, H, L, D)), vc.read(np.uint16, (B, H, L, D))
        written = np.zeros((B, L), bool)
        for r in range(R):
            b = r // Tq
            p = int(pos[r])
            # a row whose position falls outside [0, L) writes no cache
            if 0 <= p < L and lens[b] >= Tq:
                _bits_nan_aware(kg[b, :, p], k[r])
                _bits_nan_aware(vg[b, :, p], v[r])
                written[b, p] = True
        assert np.all(kg.transpose(0, 2, 1, 3)[~written] == 0xABCD)
        assert np.all(vg.transpose(0, 2, 1, 3)[~written] == 0xABCD)


def test_gemm_swiglu_random_tiles():
    """The SwiGLU-fused tile GEMM on random tiled shapes: the bits of the f32
    GEMM followed by silu_mul with group 64."""
    rng = np.random.default_rng(78)
    for i in range(6):
        n = 256 * int(rng.integers(1, 5))
        m = 128 * int(rng.integers(1, 17))
        k = 128 * int(rng.integers(1, 9))
        a = dev_normal_bf16(n * k, 800 + i, 0, 1.0)
        b = dev_normal_bf16(k * m, 800 + i, 1, 0.5)
        say(f"bf16 GEMM + SwiGLU random n={n} m={m} k={k}")
        act = ca.Buffer(n * (m // 2) * 2)
        ca.gemm_bf16_silu(a, b, act, n, m, k)
        gu = ca.Buffer(n * m * 4)
        ca.gemm_bf16(a, b, gu, n, m, k, out_f32=True)
        want = ca.Buffer(n * (m // 2) * 2)
        ca.silu_mul_bf16(gu, want, n, m // 2, 64)
        assert np.array_equal(act.read(np.uint16), want.read(np.uint16)), (n, m, k)


def test_gemm_rope_qkv_random():
    """The RoPE-fused q / k / v projection on random batches, query counts,
    head counts, cache lengths and sequence lengths: the bits of the f32
    GEMM followed by the RoPE + cache-append kernel, caches included."""
    D = 128
    rng = np.random.default_rng(79)
    for i in range(6):
        Tq = int(rng.choice([1, 2, 16, 64, 128, 256]))
        B = max(1, 256 * int(rng.integers(1, 3)) // Tq)
        H = int(rng.integers(1, 4))
        L = int(rng.integers(1, 400))
        k = 128 * int(rng.integers(1, 4))
        R, m = B * Tq, 3 * H * D
        lens = [int(x) for x in rng.integers(0, L + Tq + 5, B)]
        a = dev_normal_bf16(R * k, 900 + i, 0, 1.0)
        w = dev_normal_bf16(k * m, 900 + i, 1, 0.2)
        inv = ca.Buffer.from_array(ca.rope_inv_freq(D, 10000.0))
        tab = ca.Buffer(L * D * 4)
        ca.rope_table_f32(inv, tab, L, D)
        lb = ca.Buffer.from_array(np.array(lens, np.uint32))
        sentinel = np.full(B * H * L * D, 0xABCD, np.uint16)
        caches = [ca.Buffer.from_array(sentinel) for _ in range(4)]
        q_f, q_u = ca.Buffer(R * H * D * 2), ca.Buffer(R * H * D * 2)
        say(f"fused q/k/v + RoPE random B={B} Tq={Tq} H={H} L={L} k={k}")
        ca.gemm_bf16_rope_qkv(a, w, tab, lb, q_f, caches[0], caches[1], B, Tq, H, L, k)
        qkv = ca.Buffer(R * m * 4)
        ca.gemm_bf16(a, w, qkv, R, m, k, out_f32=True)
        ca.rope_qkv_bf16(qkv, inv, lb, q_u, caches[2], caches[3], B, Tq, H, D, L)
        assert np.array_equal(q_f.read(np.uint16), q_u.read(np.uint16)), i
        for got, want in ((caches[0], caches[2]), (caches[1], caches[3])):
            assert np.array_equal(got.read(np.uint16), want.read(np.uint16)), i


def test_embed_random():
    rng = np.random.default_rng(80)
    for i in range(6):
        V, d = 8 * int(rng.integers(1, 300)), 8 * int(rng.integers(1, 400))
        n_tok = int(rng.integers(1, 200))
        tok = rng.integers(0, V + 3, n_tok).astype(np.uint32)  # some out of range
        table = dev_normal_bf16(V * d, 1000 + i, 0)
        x = ca.Buffer(n_tok * d * 4)
        say(f"embed random V={V} d={d} tokens={n_tok}")
        ca.embed_bf16(ca.Buffer.from_array(tok), table, x, n_tok, V, d)
        got = x.read(np.float32, (n_tok, d))
        t = table.read(np.uint16, (V, d))
        ok = tok < V
        _bits_nan_aware(got[ok], oracle.bf16_bits_to_f32(t[tok[ok].astype(np.int64)]))
        assert np.all(np.isnan(got[~ok]))


def test_lm_head_argmax_random():
    """The LM-head GEMM with the argmax in its epilogue on random decode
    shapes (ragged last column block), weights with NaN entries and
    duplicated columns: logits bitwise the plain GEMM's, tokens the oracle's
    argmax of those logits."""
    rng = np.random.default_rng(81)
    for i in range(8):
        n = int(rng.integers(1, 17))
        m = 8 * int(rng.integers(16, 5000))
        k = 8 * int(rng.integers(4, 400))
        x = rng.normal(0, 1, (n, k)).astype(np.float32)
        w = rng.normal(0, 0.05, (k, m)).astype(np.float32)
        if i % 2:
            c1, c2 = sorted(rng.choice(m, 2, replace=False))
            w[:, c2] = w[:, c1] = rng.normal(0, 1, k).astype(np.float32)  # a tie between two columns
        if i % 3 == 0:
            msk = rng.random((k, m)) < 0.0003
            w[msk] = np.nan
        a = ca.Buffer.from_array(oracle.f32_to_bf16_bits_np(x))
        b = ca.Buffer.from_array(oracle.f32_to_bf16_bits_np(w))
        c, idx, plain = ca.Buffer(n * m * 4), ca.Buffer(n * 4), ca.Buffer(n * m * 4)
        say(f"LM head argmax random n={n} m={m} k={k}")
        ca.gemm_bf16_argmax(a, b, c, idx, n, m, k)
        ca.gemm_bf16(a, b, plain, n, m, k, out_f32=True)
        lg = c.read(np.float32, (n, m))
        _bits_nan_aware(lg, plain.read(np.float32, (n, m)))
        assert list(idx.read(np.uint32)) == [oracle.argmax_f32(lg[r]) for r in range(n)], i


def _mem_f32(res):
    m = res.get()
    out = ca.mem_to_array(m, np.float32)
    if m.data:
        ca.mem_free(m)
    return out


def test_runtime_programs_random():
    """The stdlib programs through Runtime::exec on seeded random inputs
    (lengths from 0): producers against their definitions, folds and softmax
    bitwise the oracle's sequential forms."""
    rt = ca.Runtime([])
    rng = np.random.default_rng(82)
    for i in range(8):
        n = int(rng.integers(0, 3000))
        x = _rows(rng, 1, max(n, 1), 0.001 if i % 2 else 0.0)[0][:n]
        v = float(np.float32(rng.normal()))
        say(f"runtime programs random n={n}")
        [r] = rt.exec("tensor.broadcast-f32", [ca.Value.f32(v), ca.Value.u64(n)], 1)
        _bits_nan_aware(_mem_f32(r), np.full(n, v, np.float32))
        [r] = rt.exec("tensor.arange-f32", [ca.Value.u64(n)], 1)
        _bits_nan_aware(_mem_f32(r), np.arange(n, dtype=np.float64).astype(np.float32))
        s0 = int(rng.integers(0, n + 1))
        ln = int(rng.integers(0, n - s0 + 1))
        [r] = rt.exec("tensor.slice-f32", [rt.mem_f32(x), ca.Value.u64(s0), ca.Value.u64(ln)], 1)
        _bits_nan_aware(_mem_f32(r), x[s0:s0 + ln])
        y = _rows(rng, 1, 1 + int(rng.integers(0, 500)), 0.0)[0]
        [r] = rt.exec("tensor.concat-f32", [rt.mem_f32(x), rt.mem_f32(y)], 1)
        _bits_nan_aware(_mem_f32(r), np.concatenate([x, y]))
        if n:
            [r] = rt.exec("sum-f32", [rt.mem_f32(x)], 1)
            _bits_nan_aware(np.float32(r.get()), np.float32(oracle.fold_sum_f32(x)))
            [r] = rt.exec("max-f32", [rt.mem_f32(x)], 1)
            _bits_nan_aware(np.float32(r.get()), np.float32(oracle.fold_max_f32(x)))
            [r] = rt.exec("nn.softmax", [rt.mem_f32(x)], 1)
            _bits_nan_aware(_mem_f32(r), oracle.softmax_f32(x))


def test_tile_gemm_paths_random():
    """Random shapes aimed at each tile path of gemm_bf16: M a multiple of
    256 with N a multiple of 128 and K a multiple of 128 (32-k kernel, wide
    or narrow tiles by the host's rule) or of 64 only (64-k kernel), and the
    same with one dimension off the tile (bounds-checked kernel): the bf16
    output within the stated bound of the sequential oracle, bitwise the RNE
    of the f32 output, and bitwise run to run."""
    from gpu_util import as_f32, bf16_ulp_of, U
    rng = np.random.default_rng(83)
    for i in range(12):
        n = 256 * int(rng.integers(1, 3))
        m = 128 * int(rng.integers(1, 9))
        k = 128 * int(rng.integers(1, 6)) if i % 3 != 1 else 64 * (2 * int(rng.integers(1, 5)) + 1)
        if i % 4 == 3:
            which = int(rng.integers(0, 3))
            n, m, k = (n + 3, m, k) if which == 0 else (n, m + 8, k) if which == 1 else (n, m, k + 8)
        a = dev_normal_bf16(n * k, 1100 + i, 0, 1.0)
        b = dev_normal_bf16(k * m, 1100 + i, 1, 1.0)
        c16, c32 = ca.Buffer(n * m * 2), ca.Buffer(n * m * 4)
        say(f"bf16 tile GEMM path random n={n} m={m} k={k}")
        ca.gemm_bf16(a, b, c16, n, m, k)
        ca.gemm_bf16(a, b, c32, n, m, k, out_f32=True)
        g16, g32 = c16.read(np.uint16, (n, m)), c32.read(np.float32, (n, m))
        assert np.array_equal(g16, oracle.f32_to_bf16_bits_np(g32)), (n, m, k)
        a16, b16 = a.read(np.uint16, (n, k)), b.read(np.uint16, (k, m))
        af, bf = as_f32(a16).astype(np.float64), as_f32(b16).astype(np.float64)
        absprod = np.abs(af) @ np.abs(bf)
        bound = 8 * (k / 32 + 1) * U * absprod
        assert np.all(np.abs(g32.astype(np.float64) - af @ bf) <= bound), (n, m, k)
        _, seq16 = oracle.matmul_bf16(a16, b16)
        g, s = as_f32(g16).astype(np.float64), as_f32(seq16).astype(np.float64)
        assert np.all(np.abs(g - s) <= bound + k * U * absprod + bf16_ulp_of(np.maximum(np.abs(g), np.abs(s))))
        ca.gemm_bf16(a, b, c16, n, m, k)
        assert np.array_equal(c16.read(np.uint16, (n, m)), g16), (n, m, k)


def test_attention_long_and_prefill_boundary_random():
    """Decode attention at random long caches (up to 6000 positions) and the
    causal form around the prefill kernel's cache limit (max_len 1,088: the
    score matrix of whole 64-key blocks fits 80 KB of LDS; the one-query
    kernel beyond it), at the limit, one past it and at random lengths:
    bitwise the oracle."""
    D = 128
    rng = np.random.default_rng(84)
    for i in range(4):
        B, H = int(rng.integers(1, 5)), int(rng.integers(1, 5))
        L = int(rng.integers(2000, 6000))
        lens = [int(x) for x in rng.integers(0, L + 1, B)]
        scale = float(np.float32(rng.uniform(0.05, 0.2)))
        q = dev_normal_bf16(B * H * D, 1200 + i, 0)
        k = dev_normal_bf16(B * H * L * D, 1200 + i, 1)
        v = dev_normal_bf16(B * H * L * D, 1200 + i, 2)
        lb, o = ca.Buffer.from_array(np.array(lens, np.uint32)), ca.Buffer(B * H * D * 4)
        say(f"attention long random B={B} H={H} L={L} lens={lens}")
        ca.attn_decode_bf16(q, k, v, lb, o, B, H, L, D, scale)
        want = oracle.attn_decode(q.read(np.uint16, (B, H, D)), k.read(np.uint16, (B, H, L, D)),
                                  v.read(np.uint16, (B, H, L, D)), np.array(lens, np.uint32), scale)
        _bits_nan_aware(o.read(np.float32, (B, H, D)), want)
    for i, L in enumerate([1088, 1089, int(rng.integers(700, 1300)), int(rng.integers(700, 1300))]):
        B, H, Tq = int(rng.integers(1, 3)), int(rng.integers(1, 3)), int(rng.integers(8, 60))
        lens = [int(x) for x in rng.integers(Tq, L + 1, B)]
        scale = float(np.float32(rng.uniform(0.05, 0.2)))
        q = dev_normal_bf16(B * Tq * H * D, 1300 + i, 0)
        k = dev_normal_bf16(B * H * L * D, 1300 + i, 1)
        v = dev_normal_bf16(B * H * L * D, 1300 + i, 2)
        lb, o = ca.Buffer.from_array(np.array(lens, np.uint32)), ca.Buffer(B * Tq * H * D * 4)
        say(f"causal attention near the prefill limit B={B} Tq={Tq} H={H} L={L} lens={lens}")
        ca.attn_causal_bf16(q, k, v, lb, o, B, Tq, H, L, D, scale, out_f32=True)
        want = od.attn_causal(q.read(np.uint16), k.read(np.uint16, (B, H, L, D)),
                              v.read(np.uint16, (B, H, L, D)), lens, B, Tq, H, D, scale)
        _bits_nan_aware(o.read(np.float32, (B * Tq, H * D)), want)


def test_bf16_gemm_special_values_random():
    """NaN, +-inf and zeros at random positions of A and B (finite values of
    moderate size, so no partial sum overflows): for every path of gemm_bf16
    (decode, tile, edge), each output is NaN exactly where the exact product
    is (a NaN input, inf * 0, or infinities of both signs in the sum),
    +-inf exactly where it is, and finite elsewhere; the bf16 output is the
    RNE of the f32 output."""
    from gpu_util import as_f32
    rng = np.random.default_rng(85)
    shapes = [(8, 1024, 512), (16, 520, 96), (256, 256, 256), (512, 384, 192), (300, 200, 100)]
    for i, (n, m, k) in enumerate(shapes):
        a = rng.normal(0, 1, (n, k)).astype(np.float32)
        b = rng.normal(0, 1, (k, m)).astype(np.float32)
        for x in (a, b):
            msk = rng.random(x.shape) < 0.0015
            x[msk] = rng.choice(np.array([np.nan, np.inf, -np.inf, 0.0], np.float32), int(msk.sum()))
        a16, b16 = oracle.f32_to_bf16_bits_np(a), oracle.f32_to_bf16_bits_np(b)
        ab, bb = ca.Buffer.from_array(a16), ca.Buffer.from_array(b16)
        c16, c32 = ca.Buffer(n * m * 2), ca.Buffer(n * m * 4)
        say(f"bf16 GEMM special values random n={n} m={m} k={k}")
        ca.gemm_bf16(ab, bb, c32, n, m, k, out_f32=True)
        ca.gemm_bf16(ab, bb, c16, n, m, k)
        g32 = c32.read(np.float32, (n, m))
        _bits_nan_aware(c16.read(np.uint16, (n, m)), oracle.f32_to_bf16_bits_np(g32))
        af, bf = as_f32(a16).astype(np.float64), as_f32(b16).astype(np.float64)
        with np.errstate(invalid="ignore", over="ignore"):
            exact = af @ bf
        assert np.array_equal(np.isnan(g32), np.isnan(exact)), (n, m, k)
        inf = np.isinf(exact)
        assert np.array_equal(np.isinf(g32), inf), (n, m, k)
        assert np.array_equal(np.sign(g32[inf]), np.sign(exact[inf])), (n, m, k)
