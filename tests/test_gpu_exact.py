"""GPU parity of the exact-order paths against the pinned oracle: bitwise.

math.exp-approx, nn.softmax and the f32 matmul contraction reproduce the
reference's operation order exactly, so every output bit must match the CPU
oracle on the same inputs (NaN payloads excepted: only NaN-ness is compared).
"""
import json
import os

import numpy as np
import pytest

import catena_amd as ca
import oracle
from gpu_util import hash_bits, say

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_known_answers.json")))


@pytest.fixture(scope="module", autouse=True)
def _init():
    say("init device 0")
    ca.init(0)


def _bits_equal_nan_aware(x: np.ndarray, y: np.ndarray) -> bool:
    xn, yn = np.isnan(x), np.isnan(y)
    if not np.array_equal(xn, yn):
        return False
    return np.array_equal(x[~xn].view(np.uint32), y[~yn].view(np.uint32))


def test_exp_approx_bitwise_sweep():
    rng = np.random.default_rng(21)
    x = np.concatenate([
        np.linspace(-100, 100, 400001).astype(np.float32),
        rng.integers(0, 2 ** 32, 600000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 88.5, -88.5, 89.5, -89.5, 1e-40, -1e-40],
                 np.float32),
    ]).astype(np.float32)
    say(f"exp-approx sweep n={x.size}")
    xb, yb = ca.Buffer.from_array(x), ca.Buffer(x.nbytes)
    ca.exp_approx_f32(xb, yb, x.size)
    got = yb.read(np.float32)
    L = oracle.lib()
    want = np.array([L.or_exp_approx(float(v)) for v in x], np.float32)
    assert _bits_equal_nan_aware(got, want)


_MAP = {  # catena_map_op_t -> oracle name
    ca.MAP_EXP_APPROX: "exp_approx", ca.MAP_SQRT: "sqrt_newton", ca.MAP_SIGMOID: "sigmoid",
    ca.MAP_SILU: "silu", ca.MAP_SIN_APPROX: "sin_approx", ca.MAP_COS_APPROX: "cos_approx",
    ca.MAP_SIN_APPROX_FULL: "sin_full",
}


@pytest.mark.parametrize("op", sorted(_MAP), ids=[_MAP[k] for k in sorted(_MAP)])
def test_scalar_map_bitwise_sweep(op):
    """Each scalar stdlib program elementwise on the GPU against the pinned
    oracle, bit for bit: 2M random bit patterns, a dense sweep of [-300, 300]
    and the special values."""
    rng = np.random.default_rng(100 + op)
    x = np.concatenate([
        np.linspace(-300, 300, 1_000_001).astype(np.float32),
        rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 3.4e38, -3.4e38],
                 np.float32),
    ]).astype(np.float32)
    say(f"scalar map {_MAP[op]} sweep n={x.size}")
    xb, yb = ca.Buffer.from_array(x), ca.Buffer(x.nbytes)
    ca.map_f32(op, xb, yb, x.size)
    assert _bits_equal_nan_aware(yb.read(np.float32), oracle.map_f32(_MAP[op], x))
    # in place (y == x)
    ca.map_f32(op, xb, xb, x.size)
    assert _bits_equal_nan_aware(xb.read(np.float32), oracle.map_f32(_MAP[op], x))


def test_runtime_scalar_programs_reference_tests():
    """math.sqrt, nn.sigmoid, nn.silu, math.sin-approx, math.cos-approx and
    math.sin-approx-full through Runtime::exec (built-in stdlib programs,
    (f32) -> (f32)): bitwise the oracle, and within the reference's own
    tolerance on its own test inputs (fixtures cite catena-lang/tests/
    runtime.rs)."""
    rt = ca.Runtime([])
    cases = [("math.sqrt", "sqrt_newton", "sqrt"), ("nn.sigmoid", "sigmoid", "sigmoid"),
             ("nn.silu", "silu", "silu"), ("math.sin-approx", "sin_approx", "sin_approx"),
             ("math.sin-approx-full", "sin_full", "sin_approx_full"),
             ("math.cos-approx", "cos_approx", None)]
    for program, name, key in cases:
        g = GOLDEN[key] if key else {"inputs": [0.0, 0.5, 1.0, -0.5, -1.0]}
        for i, v in enumerate(g["inputs"]):
            say(f"runtime exec {program}({v})")
            [r] = rt.exec(program, [ca.Value.f32(v)], 1)
            assert r.kind == ca.KIND_F32
            want = oracle.scalar(name, v)
            assert np.float32(r.get()).view(np.uint32) == np.float32(want).view(np.uint32), (program, v)
            if key:
                assert abs(r.get() - g["expected"][i]) < g["absolute_tolerance"], (program, v)
            else:  # math.cos-approx has no reference test: libm on its Taylor range
                assert abs(r.get() - np.cos(v)) < 1e-3, (program, v)
    rt.close()


@pytest.mark.parametrize("n", [1, 2, 3, 255, 256, 257, 4096, 100003])
def test_softmax_bitwise(n):
    rng = np.random.default_rng(n)
    x = (rng.normal(0, 4, n)).astype(np.float32)
    say(f"softmax n={n}")
    xb, yb = ca.Buffer.from_array(x), ca.Buffer(x.nbytes)
    ca.softmax_f32(xb, yb, 1, n)
    assert np.array_equal(yb.read(np.float32).view(np.uint32), oracle.softmax_f32(x).view(np.uint32))


def test_softmax_rows_in_place_and_specials():
    rows = [
        np.array([1.0, 2.0, 4.0, 0.5], np.float32),
        np.array([0.0, -0.0, -0.0, 0.0], np.float32),           # max tie: first (+0) wins
        np.array([-0.0, 0.0, 0.0, -0.0], np.float32),           # first (-0) wins
        np.array([5.0, np.nan, 1.0, 2.0], np.float32),          # NaN resets the max fold
        np.array([1.0, 2.0, 3.0, np.nan], np.float32),          # trailing NaN is the max
        np.array([-np.inf, -np.inf, -np.inf, -np.inf], np.float32),
        np.array([3.0, 3.0, 3.0, 3.0], np.float32),
        np.array([100.0, -100.0, 50.0, 89.0], np.float32),      # exp~ wrap region
    ]
    x = np.stack(rows)
    say("softmax rows specials (in place)")
    buf = ca.Buffer.from_array(x)
    ca.softmax_f32(buf, buf, x.shape[0], x.shape[1])
    got = buf.read(np.float32, x.shape)
    for i, r in enumerate(rows):
        assert _bits_equal_nan_aware(got[i], oracle.softmax_f32(r)), i


@pytest.mark.parametrize("n,m,k", [(256, 256, 256), (1, 1, 1), (65, 33, 17), (130, 70, 300),
                                   (64, 64, 0), (3, 200, 5), (257, 129, 64), (100, 77, 131),
                                   # 16x16 tiles with A by DPP row broadcast (k % 16 == 0,
                                   # m % 4 == 0): ragged rows and column blocks, one to
                                   # three chunks of 256 k, a last chunk of 1 to 16 groups
                                   (255, 196, 320), (3, 4, 64), (130, 260, 512), (257, 300, 576),
                                   (1, 64, 128), (61, 1000, 192), (33, 20, 48), (100, 36, 272),
                                   # 64x64 tiles (at least 256 of them)
                                   (1040, 1030, 37), (1024, 1024, 130)])
def test_gemm_f32_exact_bitwise(n, m, k):
    rng = np.random.default_rng(n + m + k)
    a = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, m)).astype(np.float32)
    say(f"gemm f32 exact {n}x{m}x{k}")
    ab, bb, cb = ca.Buffer.from_array(a), ca.Buffer.from_array(b), ca.Buffer(n * m * 4)
    ca.gemm_f32_exact(ab, bb, cb, n, m, k)
    got = cb.read(np.float32, (n, m))
    want = oracle.matmul_f32(a, b) if k else np.zeros((n, m), np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gemm_f32_exact_tile_instances_agree():
    """Rows 256..511 of a 1024 x 1024 x 300 product (64x64 tiles: 256 of
    them) computed alone as a 256 x 1024 product (16x16 tiles: 64 tiles of
    64x64 would leave CUs idle): the same bits, since every cell is one
    k-ascending chain in both instances."""
    n, m, k = 1024, 1024, 300
    rng = np.random.default_rng(77)
    a = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, m)).astype(np.float32)
    ab, bb = ca.Buffer.from_array(a), ca.Buffer.from_array(b)
    full, part = ca.Buffer(n * m * 4), ca.Buffer(256 * m * 4)
    say("gemm f32 exact 1024x1024x300 (64x64 tiles) and rows 256..511 alone (16x16 tiles)")
    ca.gemm_f32_exact(ab, bb, full, n, m, k)
    ca.gemm_f32_exact(ca.Buffer.from_array(np.ascontiguousarray(a[256:512])), bb, part, 256, m, k)
    assert np.array_equal(full.read(np.uint32, (n, m))[256:512], part.read(np.uint32, (256, m)))


def test_gemm_f32_exact_dpp_instance_agrees_and_specials():
    """Rows 256..511 of a 1024 x 1024 x 320 product (64x64 tiles) computed
    alone as a 256 x 1024 product (16x16 tiles with A by DPP row broadcast:
    k % 16 == 0, m % 4 == 0): the same bits.  Then special values through
    that instance and the all-LDS 16x16 one (m % 4 != 0) against the oracle:
    signed zeros, infinities, NaNs and products below the normal range."""
    n, m, k = 1024, 1024, 320
    rng = np.random.default_rng(78)
    a = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, m)).astype(np.float32)
    ab, bb = ca.Buffer.from_array(a), ca.Buffer.from_array(b)
    full, part = ca.Buffer(n * m * 4), ca.Buffer(256 * m * 4)
    say("gemm f32 exact 1024x1024x320 (64x64 tiles) and rows 256..511 alone (DPP 16x16 tiles)")
    ca.gemm_f32_exact(ab, bb, full, n, m, k)
    ca.gemm_f32_exact(ca.Buffer.from_array(np.ascontiguousarray(a[256:512])), bb, part, 256, m, k)
    assert np.array_equal(full.read(np.uint32, (n, m))[256:512], part.read(np.uint32, (256, m)))
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-20, -1e-20, 3e-39, 1.0, -2.5],
                        np.float32)
    for (n, m, k) in [(66, 132, 128), (66, 131, 128)]:  # DPP instance; all-LDS instance
        a = rng.uniform(-1, 1, (n, k)).astype(np.float32)
        b = rng.uniform(-1, 1, (k, m)).astype(np.float32)
        ai = rng.random((n, k)) < 0.01
        a[ai] = rng.choice(specials, int(ai.sum()))
        bi = rng.random((k, m)) < 0.01
        b[bi] = rng.choice(specials, int(bi.sum()))
        b[:, :3] *= np.float32(1e-19)  # products below the normal range in three columns
        say(f"gemm f32 exact specials {n}x{m}x{k}")
        cb = ca.Buffer(n * m * 4)
        ca.gemm_f32_exact(ca.Buffer.from_array(a), ca.Buffer.from_array(b), cb, n, m, k)
        got = cb.read(np.float32, (n, m))
        want = oracle.matmul_f32(a, b)
        assert _bits_equal_nan_aware(got, want)


def test_gemm_f32_exact_random_shapes_all_instances():
    """40 seeded random shapes spread over the three instances (64x64 tiles,
    16x16 tiles through LDS, 16x16 tiles with A by DPP row broadcast) and
    their edges (k = 16, m = 4, one row, one column, k a multiple of 16 but
    not of 256): every cell bitwise the oracle's ascending chain."""
    rng = np.random.default_rng(2024)
    shapes = [(1, 4, 16), (17, 8, 16), (16, 16, 16), (2, 4, 4096), (300, 4, 32)]
    while len(shapes) < 40:
        n = int(rng.integers(1, 400))
        m = int(rng.integers(1, 400))
        k = int(rng.integers(0, 700))
        if rng.random() < 0.5:
            m = max(4, m - m % 4)      # 16-byte rows of B
            k = 16 * (k // 16)         # the DPP instance's k
        shapes.append((n, m, k))
    for (n, m, k) in shapes:
        a = rng.uniform(-1, 1, (n, k)).astype(np.float32)
        b = rng.uniform(-1, 1, (k, m)).astype(np.float32)
        say(f"gemm f32 exact random shape {n}x{m}x{k}")
        cb = ca.Buffer(max(1, n * m) * 4)
        ca.gemm_f32_exact(ca.Buffer.from_array(a) if a.size else ca.Buffer(4),
                          ca.Buffer.from_array(b) if b.size else ca.Buffer(4), cb, n, m, k)
        got = cb.read(np.float32, (n, m))
        want = oracle.matmul_f32(a, b) if k else np.zeros((n, m), np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n, m, k)


def test_gemm_f32_exact_run_to_run():
    n = m = k = 256
    a = ca.Buffer(n * k * 4)
    b = ca.Buffer(k * m * 4)
    ca.fill_uniform_f32(a, n * k, 1, 0)
    ca.fill_uniform_f32(b, k * m, 2, 0)
    c = ca.Buffer(n * m * 4)
    say("gemm f32 exact run-to-run x10")
    hashes = set()
    for _ in range(10):
        ca.gemm_f32_exact(a, b, c, n, m, k)
        hashes.add(hash_bits(c.read(np.uint32)))
    assert len(hashes) == 1
    # and against the oracle on the device-generated inputs
    want = oracle.matmul_f32(a.read(np.float32, (n, k)), b.read(np.float32, (k, m)))
    assert np.array_equal(c.read(np.uint32, (n, m)), want.view(np.uint32))


# ---------------------------------------------------------------- runtime / programs
MATMUL_DECLS = """
(def program matmul-2x2-via-mem :
  ([n m k.] {(cap.ref mem) (cap.ref mem) ({[.n] u64} :) ({[.m] u64} :) ({[.k] u64} :)
             ({({[.n] [.k]} *) u64} :) ({({[.k] [.m]} *) u64} :) ({({[.n] [.m]} *) u64} :)})
  -> ([n m k.] (cap.own mem)) = native)
(def program matmul-right-identity-2x2-via-mem :
  ([n.] {(cap.ref mem) ({[.n] u64} :) ({({[.n] [.n]} *) u64} :)}) -> ([n.] (cap.own mem)) = native)
(def program matmul-left-identity-2x2-via-mem :
  ([n.] {(cap.ref mem) ({[.n] u64} :) ({({[.n] [.n]} *) u64} :)}) -> ([n.] (cap.own mem)) = native)
"""


def test_runtime_matmul_reference_known_answer():
    g = GOLDEN["matmul_2x2_via_mem"]
    rt = ca.Runtime([MATMUL_DECLS])
    a, b = rt.mem_f32(g["a"]), rt.mem_f32(g["b"])
    say("runtime exec matmul-2x2-via-mem")
    [res] = rt.exec("matmul-2x2-via-mem",
                    [a, b] + [ca.Value.u64(g[x]) for x in ("n", "m", "k", "nk", "km", "nm")], 1)
    assert res.kind == ca.KIND_MEM
    vals = ca.mem_to_array(res.get(), np.float32)
    assert np.abs(vals - np.array(g["expected"], np.float32)).max() < g["tolerance"]
    assert vals.tolist() == g["expected"]
    for v in (a, b, res):
        ca.mem_free(v.get())


def test_runtime_identity_programs_exact():
    g = GOLDEN["matmul_identity"]
    rt = ca.Runtime([MATMUL_DECLS])
    for name in ("matmul-right-identity-2x2-via-mem", "matmul-left-identity-2x2-via-mem"):
        a = rt.mem_f32(g["a"])
        say(f"runtime exec {name}")
        [res] = rt.exec(name, [a, ca.Value.u64(g["n"]), ca.Value.u64(g["nn"])], 1)
        assert ca.mem_to_array(res.get(), np.float32).tolist() == g["expected"]
        ca.mem_free(a.get())
        ca.mem_free(res.get())


def test_runtime_softmax_and_exp_reference_tests():
    rt = ca.Runtime([])
    g = GOLDEN["softmax"]
    x = rt.mem_f32(g["input"])
    say("runtime exec nn.softmax")
    [res] = rt.exec("nn.softmax", [x], 1)
    vals = ca.mem_to_array(res.get(), np.float32)
    xin = np.array(g["input"], np.float64)
    e = np.exp(xin - xin.max())
    assert np.abs(vals - e / e.sum()).max() < g["absolute_tolerance"]
    assert abs(vals.astype(np.float64).sum() - 1.0) < g["sum_tolerance"]
    assert np.array_equal(vals, oracle.softmax_f32(np.array(g["input"], np.float32)))
    ge = GOLDEN["exp_approx"]
    for v in ge["inputs"]:
        say(f"runtime exec math.exp-approx({v})")
        [r] = rt.exec("math.exp-approx", [ca.Value.f32(v)], 1)
        assert r.kind == ca.KIND_F32
        assert np.float32(r.get()).view(np.uint32) == np.float32(oracle.exp_approx(v)).view(np.uint32)
        assert abs(r.get() - np.exp(v)) / max(np.exp(v), 1.0) < ge["relative_tolerance"]


def test_copy_kernel():
    x = np.random.default_rng(1).integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    src, dst = ca.Buffer.from_array(x), ca.Buffer(x.nbytes)
    say("copy kernel 4 MiB")
    ca.copy_bytes(dst, src, x.nbytes)
    assert np.array_equal(dst.read(np.uint32), x)


def test_pool_reuses_blocks():
    before = ca.pool_stats()["device_allocs"]
    for _ in range(50):
        b = ca.Buffer(1 << 20)
        b.close()
    assert ca.pool_stats()["device_allocs"] - before <= 1


def test_program_matmul_via_mem_c1_by_value():
    """C1: the 256^3 f32 GEMM through the program ABI symbol itself,
    program_matmul_2x2_via_mem, called the way the reference's libffi
    executor calls a generated program (catena-lang/src/runtime/
    executor.rs:88-106: each Mem argument by value as a 16-byte struct, the
    u64 sizes by value, one pointer per output), on U[-1,1] inputs from seeds
    1 and 2: bitwise equal to the oracle, and bitwise run to run."""
    import ctypes
    n = m = k = 256
    a, b = ca.Buffer(n * k * 4), ca.Buffer(k * m * 4)
    ca.fill_uniform_f32(a, n * k, 1, 0)
    ca.fill_uniform_f32(b, k * m, 2, 0)
    a_host, b_host = a.read(np.float32, (n, k)), b.read(np.float32, (k, m))
    assert a_host.min() >= -1 and a_host.max() <= 1 and np.unique(a_host).size > 60000
    want = oracle.matmul_f32(a_host, b_host).view(np.uint32)
    L = ca.lib()
    hashes = set()
    for i in range(5):
        out = ca.Mem()
        say(f"program_matmul_2x2_via_mem 256^3 by value, call {i}")
        L.program_matmul_2x2_via_mem(a.mem, b.mem, n, m, k, n * k, k * m, n * m, ctypes.byref(out))
        assert out.len == n * m * 4 and out.data
        got = ca.mem_to_array(out, np.uint32).reshape(n, m)
        assert np.array_equal(got, want)
        hashes.add(hash_bits(got))
        ca.mem_free(out)
    assert len(hashes) == 1
