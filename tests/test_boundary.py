"""CPU checks of the drop-in boundary that need no GPU.

* Fail-stop: the program ABI traps on a failed length assertion before any
  device call, like the reference's generated module (catena_assert:
  message on stderr, then a trap; catena-lang/src/codegen/prelude.rs:38-55),
  for the assertions of tests/cases/matrix/matmul.hex:16-29.  Each case runs
  in a child process, which must die of SIGILL / SIGTRAP with the message.
* The reference's own sources: feeding the stdlib and test-case .hex files
  of the reference checkout (when one is present; skipped otherwise) to
  catena_runtime_from_sources, the way Runtime::from_sources takes
  stdlib::sources() plus a test's program (catena-lang/src/stdlib.rs:47-66),
  binds every hot program with the reference's declared kinds.
* The decode GEMM's k split is a function of the shape alone.
* Size limits rejected before any device call.
"""
import glob
import os
import signal
import subprocess
import sys
import textwrap

import pytest

import catena_amd as ca

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference/catena-lang"

_CHILD = textwrap.dedent("""
    import ctypes, sys
    sys.path.insert(0, {pkg!r})
    import catena_amd as ca
    L = ca.lib()
    a = ca.Mem(); a.data = 16; a.len = {alen}
    b = ca.Mem(); b.data = 32; b.len = {blen}
    out = ca.Mem()
    print("calling", flush=True)
    L.program_matmul_2x2_via_mem(a, b, {n}, {m}, {k}, {nk}, {km}, {nm}, ctypes.byref(out))
    print("returned", flush=True)
""")


def _run_child(**kw):
    code = _CHILD.format(pkg=os.path.join(ROOT, "catena-lang_amd"), **kw)
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)


@pytest.mark.parametrize("case,msg", [
    # nk != len(a) / 4: a holds 2x3 f32 = 24 bytes, nk claims 8 elements
    (dict(alen=24, blen=24, n=2, m=2, k=3, nk=8, km=6, nm=4), "nk == len(a)"),
    # km != len(b) / 4
    (dict(alen=24, blen=20, n=2, m=2, k=3, nk=6, km=6, nm=4), "km == len(b)"),
    # lengths agree with nk / km, but n * k != nk (the value-level check)
    (dict(alen=24, blen=24, n=3, m=2, k=3, nk=6, km=6, nm=4), "n*k == nk"),
])
def test_program_matmul_traps_on_failed_assertion(case, msg):
    """The assertion fires before any device call (the pointers here are not
    device memory and are never dereferenced), so this runs without a GPU."""
    r = _run_child(**case)
    assert "calling" in r.stdout and "returned" not in r.stdout
    assert r.returncode in (-signal.SIGILL, -signal.SIGTRAP), (r.returncode, r.stderr[-500:])
    assert "catena assertion failed" in r.stderr and msg in r.stderr, r.stderr[-500:]


def _ref_sources():
    files = sorted(glob.glob(os.path.join(REF, "stdlib", "*.hex")))
    cases = sorted(glob.glob(os.path.join(REF, "tests", "cases", "**", "*.hex"), recursive=True))
    return files, cases


# hot programs with the kinds the reference declares for them
# (catena-lang/stdlib/*.hex, catena-lang/tests/cases/{matrix,reducec}/*.hex)
_U64, _F32, _MEM = ca.KIND_U64, ca.KIND_F32, ca.KIND_MEM
HOT = {
    "matmul-2x2-via-mem": ([_MEM, _MEM] + [_U64] * 6, 1),
    "matmul-right-identity-2x2-via-mem": ([_MEM, _U64, _U64], 1),
    "matmul-left-identity-2x2-via-mem": ([_MEM, _U64, _U64], 1),
    "nn.softmax": ([_MEM], 1),
    "math.exp-approx": ([_F32], 1),
    "math.sqrt": ([_F32], 1),
    "nn.sigmoid": ([_F32], 1),
    "nn.silu": ([_F32], 1),
    "math.sin-approx": ([_F32], 1),
    "math.cos-approx": ([_F32], 1),
    "math.sin-approx-full": ([_F32], 1),
    "nn.rmsnorm": ([_MEM], 1),
    "tensor.argmax-f32": ([_MEM], 1),
    "tensor.broadcast-f32": ([_F32, _U64], 1),
    "tensor.arange-f32": ([_U64], 1),
    "tensor.slice-f32": ([_MEM, _U64, _U64], 1),
    "tensor.concat-f32": ([_MEM, _MEM], 1),
    "sum-f32": ([_MEM], 1),
    "mean-f32": ([_MEM], 1),
    "max-f32": ([_MEM], 1),
    "sum-u64": ([_MEM], 1),
    "dot-u64": ([_MEM, _MEM], 1),
}


def _value_of(kind):
    return {ca.KIND_U64: ca.Value.u64(1), ca.KIND_F32: ca.Value.f32(1.0),
            ca.KIND_MEM: ca.Value.mem(ca.Mem()), ca.KIND_U32: ca.Value.u32(1),
            ca.KIND_BOOL: ca.Value.bool(True)}[kind]


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "stdlib")),
                    reason="no reference checkout in this environment")
def test_reference_sources_bind_every_hot_program():
    stdlib, cases = _ref_sources()
    assert len(stdlib) >= 10 and cases
    texts = [open(p).read() for p in stdlib + cases]
    rt = ca.Runtime(texts)
    names = set(rt.programs())
    missing = [n for n in HOT if n not in names]
    assert not missing, missing
    # The declared kinds: for each input position, a value of a different
    # kind there (all others right) is refused with TypeMismatch naming that
    # index and the declared kind.  Validation fails before any call, so no
    # device is touched.
    for name, (kinds, n_out) in HOT.items():
        for i, want in enumerate(kinds):
            args = [_value_of(k) for k in kinds]
            args[i] = ca.Value.bool(True)
            with pytest.raises(ca.ExecError) as e:
                rt.exec(name, args, n_out)
            assert (e.value.status, e.value.index, e.value.expected, e.value.actual) == (
                ca.EXEC_TYPE_MISMATCH, i, want, ca.KIND_BOOL), (name, i)
        # one input too many: input arity names the declared count
        with pytest.raises(ca.ExecError) as e:
            rt.exec(name, [_value_of(k) for k in kinds] + [ca.Value.u64(0)], n_out)
        assert (e.value.status, e.value.expected) == (ca.EXEC_INPUT_ARITY_MISMATCH, len(kinds))


def test_decode_split_depends_on_shape_only():
    """The k split (and so which partial sums are added) is a function of
    (n, m, k): no device is initialised here, and the values are those of
    the rule stated in kernels.cpp for 256 spread slots."""
    cases = {
        # (n, m, k): (k groups, partial bytes)
        (16, 11008, 4096): (2, 2 * 16 * 11008 * 4),
        (16, 4096, 11008): (8, 8 * 16 * 4096 * 4),
        (8, 6144, 2048): (2, 2 * 8 * 6144 * 4),     # C5 W_qkv
        (8, 2048, 2048): (8, 8 * 8 * 2048 * 4),     # C5 W_o: 16 MiB weight, 2 steps per wave
        (8, 11264, 2048): (2, 2 * 8 * 11264 * 4),   # C5 W_gu
        (8, 2048, 5632): (6, 6 * 8 * 2048 * 4),     # C5 W_down
        (8, 32000, 2048): (1, 0),                   # C5 LM head: no split
        (16, 4096, 2056): (9, 9 * 16 * 4096 * 4),   # register path (k % 32 != 0)
    }
    for (n, m, k), want in cases.items():
        assert ca.gemm_bf16_decode_plan(n, m, k) == want, (n, m, k)
    # partial bytes scale with n only: the split itself ignores the row count
    for n in range(1, 17):
        g, nbytes = ca.gemm_bf16_decode_plan(n, 11008, 4096)
        assert g == 2 and nbytes == 2 * n * 11008 * 4
    with pytest.raises(ca.CatenaError):
        ca.gemm_bf16_decode_plan(17, 128, 128)
    with pytest.raises(ca.CatenaError):
        ca.gemm_bf16_decode_plan(4, 100, 128)


def test_sum_rows_longer_than_the_fold_bound_are_rejected():
    """sum-f32 / mean-f32 rows are folded in 32-bit chunks of 2048 values:
    rows past 0xFFFFF800 elements are refused before any device call (the
    pointers here are never dereferenced)."""
    L = ca.lib()
    for f in (L.catena_mi355x_sum_f32, L.catena_mi355x_mean_f32):
        assert f(16, 32, 1, 0xFFFFF801) == 2   # CATENA_ERR_UNSUPPORTED
        assert f(16, 32, 1, 1 << 32) == 2
        # at the bound the shape is accepted and the call proceeds to device
        # set-up (which, without a GPU, reports NOT_INITIALIZED)
        st = f(16, 32, 1, 0xFFFFF800)
        assert st in (0, 5)
