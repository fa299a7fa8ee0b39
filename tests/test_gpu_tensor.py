"""GPU parity of the buffer producers and folds: the reference's
tensor.broadcast-f32 / arange-f32 / slice-f32 / concat-f32 and sum-f32 /
mean-f32 / max-f32 (stdlib), sum-u64 / dot-u64 (its reducec test programs).

The reference's own test vectors run through Runtime::exec (fixture
tests/golden/reference_known_answers.json); larger inputs are checked
against the oracle's sequential folds bit for bit, arange against numpy's
round-to-nearest u64 -> f32 conversion, and the u64 folds against numpy's
wrapping uint64 arithmetic.
"""
import json
import os

import numpy as np
import pytest

import catena_amd as ca
import oracle
from gpu_util import say

pytestmark = pytest.mark.gpu

G = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))

U64_DECL = """
# declarations of the reference's reducec test programs (tests/cases/reducec/basic.hex)
(def program sum-u64 : (cap.ref mem) -> (u64 val) = native)
(def program dot-u64 : {(cap.ref mem) (cap.ref mem)} -> (u64 val) = native)
"""


@pytest.fixture(scope="module", autouse=True)
def _init():
    say("init device 0")
    ca.init(0)


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _mem_result(res):
    m = res.get()
    out = ca.mem_to_array(m, np.float32)
    if m.data:
        ca.mem_free(m)
    return out


def test_reference_producer_cases():
    rt = ca.Runtime([])
    t = G["tensor_producers"]
    for c in t["broadcast"]:
        say(f"tensor.broadcast-f32 {c}")
        [r] = rt.exec("tensor.broadcast-f32", [ca.Value.f32(c["value"]), ca.Value.u64(c["len"])], 1)
        assert list(_mem_result(r)) == c["expected"]
    for c in t["arange"]:
        say(f"tensor.arange-f32 {c}")
        [r] = rt.exec("tensor.arange-f32", [ca.Value.u64(c["len"])], 1)
        assert list(_mem_result(r)) == c["expected"]
    for c in t["slice"]:
        say(f"tensor.slice-f32 {c}")
        [r] = rt.exec("tensor.slice-f32", [rt.mem_f32(c["input"]), ca.Value.u64(c["start"]),
                                           ca.Value.u64(c["len"])], 1)
        assert list(_mem_result(r)) == c["expected"]
    for c in t["concat"]:
        say(f"tensor.concat-f32 {c}")
        [r] = rt.exec("tensor.concat-f32", [rt.mem_f32(c["left"]), rt.mem_f32(c["right"])], 1)
        assert list(_mem_result(r)) == c["expected"]


def test_reference_fold_cases():
    rt = ca.Runtime([U64_DECL])
    c = G["sum_mean_max_f32"]
    for name, key in [("sum-f32", "sum"), ("mean-f32", "mean"), ("max-f32", "max")]:
        say(f"{name} {c['input']}")
        [r] = rt.exec(name, [rt.mem_f32(c["input"])], 1)
        assert r.get() == c[key]
    u = G["reducec_u64"]
    say("sum-u64 / dot-u64")
    [r] = rt.exec("sum-u64", [rt.mem_u64(u["sum_u64"]["input"])], 1)
    assert r.get() == u["sum_u64"]["expected"]
    [r] = rt.exec("dot-u64", [rt.mem_u64(u["dot_u64"]["lhs"]), rt.mem_u64(u["dot_u64"]["rhs"])], 1)
    assert r.get() == u["dot_u64"]["expected"]


@pytest.mark.parametrize("rows,n", [(1, 1), (3, 1000), (2, 4097), (1, 1 << 20), (5, 31)])
def test_sum_mean_max_rows_bitwise(rows, n):
    rng = np.random.default_rng(n + rows)
    x = (rng.standard_normal((rows, n)) * np.exp(rng.uniform(-8, 8, (rows, n)))).astype(np.float32)
    if n > 40:
        x[0, 7] = -0.0
        x[-1, n // 3] = np.inf
    xb = ca.Buffer.from_array(x)
    o = ca.Buffer(rows * 4)
    say(f"sum/mean/max rows={rows} n={n}")
    ca.sum_f32(xb, o, rows, n)
    s = o.read(np.float32)
    assert np.array_equal(_bits(s), _bits([oracle.fold_sum_f32(r) for r in x]))
    ca.mean_f32(xb, o, rows, n)
    m = o.read(np.float32)
    want = [np.float32(oracle.fold_sum_f32(r)) / np.float32(n) for r in x]
    assert np.array_equal(_bits(m), _bits(want))
    ca.max_f32(xb, o, rows, n)
    mx = o.read(np.float32)
    assert np.array_equal(_bits(mx), _bits([oracle.fold_max_f32(r) for r in x]))


def test_max_nan_and_zero_cases():
    nan, inf = np.nan, np.inf
    rows = [[1.0, nan, 0.5, 0.7], [1.0, 2.0, 3.0, nan], [-0.0, 0.0, -1.0, -0.0], [0.0, -0.0, -1.0, 0.0],
            [-inf, -inf, -inf, -inf], [nan, nan, nan, 3.0]]
    x = np.array(rows, np.float32)
    o = ca.Buffer(len(rows) * 4)
    say("max-f32 NaN / signed zero rows")
    ca.max_f32(ca.Buffer.from_array(x), o, len(rows), 4)
    got = o.read(np.float32)
    want = np.array([oracle.fold_max_f32(r) for r in x], np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(_bits(got[ok]), _bits(want[ok]))


def test_empty_folds():
    rt = ca.Runtime([])
    say("sum/max of an empty buffer")
    [r] = rt.exec("sum-f32", [rt.mem_f32([])], 1)
    assert _bits([r.get()])[0] == 0          # +0: the fold never runs
    [r] = rt.exec("max-f32", [rt.mem_f32([])], 1)
    assert r.get() == -np.inf
    [r] = rt.exec("mean-f32", [rt.mem_f32([])], 1)
    assert np.isnan(r.get())                 # 0 / 0: the reference leaves it to the caller


def test_arange_beyond_2_pow_24_and_broadcast_copy():
    n = (1 << 24) + 12345
    out = ca.Buffer(n * 4)
    say(f"arange n={n}")
    ca.arange_f32(out, n)
    got = out.read(np.float32)
    assert np.array_equal(_bits(got), _bits(np.arange(n, dtype=np.uint64).astype(np.float32)))
    say("broadcast + copy at odd offsets")
    ca.broadcast_f32(out, 1000, -2.5)
    assert np.all(out.read(np.float32, (1000,)) == -2.5)
    src = ca.Buffer.from_array(np.arange(100, dtype=np.float32))
    dst = ca.Buffer(400)
    ca.copy_f32(dst.ptr + 4, src.ptr + 12, 37)
    d = dst.read(np.float32)
    assert np.array_equal(d[1:38], np.arange(3, 40, dtype=np.float32))


def test_u64_folds_wrap():
    rng = np.random.default_rng(5)
    a = rng.integers(0, 2 ** 63, (3, 5000), dtype=np.uint64) * np.uint64(3)
    b = rng.integers(0, 2 ** 63, (3, 5000), dtype=np.uint64)
    ab, bb, o = ca.Buffer.from_array(a), ca.Buffer.from_array(b), ca.Buffer(3 * 8)
    say("sum-u64 / dot-u64 rows with wraparound")
    ca.sum_u64(ab, o, 3, 5000)
    with np.errstate(over="ignore"):
        assert np.array_equal(o.read(np.uint64), a.sum(axis=1, dtype=np.uint64))
        ca.dot_u64(ab, bb, o, 3, 5000)
        assert np.array_equal(o.read(np.uint64), (a * b).sum(axis=1, dtype=np.uint64))
