"""CPU checks of the C-ABI library: it loads, exports every symbol the header
declares, ships its gfx950 code objects, keeps the no-FMA contract in the
exact-order kernels, and the runtime mirror validates like the reference's
Runtime::exec (catena-lang/src/runtime/runtime.rs:175-236) -- all without a
GPU (no compute call is made here)."""
import os
import re
import shutil
import subprocess

import pytest

import catena_amd as ca

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "catena_mi355x.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:catena|program)_\w+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    L = ca.lib()
    names = header_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # and the binding declares exactly the header's surface
    assert sorted(ca.SIGNATURES) == names


def test_code_objects_present_and_gfx950():
    objdump = "/opt/rocm/llvm/bin/llvm-readelf"
    for name in ["gemm_f32_exact", "gemm_bf16", "gemm_bf16_lds", "gemm_bf16_k32", "gemm_bf16_decode",
                 "attn_decode", "attn_prefill", "block", "tensor", "softmax", "fill"]:
        path = os.path.join(ca.LIB_DIR, name + ".co")
        assert os.path.exists(path), path
        if os.path.exists(objdump):
            out = subprocess.run([objdump, "-h", "--notes", path], capture_output=True, text=True).stdout
            assert "gfx950" in out


def _disasm(name):
    tool = "/opt/rocm/llvm/bin/llvm-objdump"
    if not os.path.exists(tool):
        pytest.skip("llvm-objdump not available")
    return subprocess.run([tool, "-d", "--mcpu=gfx950", os.path.join(ca.LIB_DIR, name + ".co")],
                          capture_output=True, text=True, check=True).stdout


FLOAT_FMA = re.compile(r"\b(v_fma_f32|v_fmac_f32\w*|v_mad_f32|v_mac_f32\w*|v_pk_fma_f32|v_fma_mix\w*|v_pk_mul_f32|v_pk_add_f32)\b")


def test_exact_gemm_has_no_float_fma():
    """The exact-order GEMM must be v_mul_f32 + v_add_f32 chains only
    (reference flags -ffp-contract=off, catena-lang/src/runtime/artifact.rs:59-71)."""
    text = _disasm("gemm_f32_exact")
    assert not FLOAT_FMA.findall(text)
    assert "v_mul_f32" in text and "v_add_f32" in text


def test_attention_fma_only_inside_division():
    """In the attention, softmax and decoder-block kernels the only fused ops are the ones of
    the correctly rounded f32 division sequence (v_div_scale / v_rcp / fma
    refinement / v_div_fmas / v_div_fixup): every function with a float FMA
    also has a v_div_fixup_f32, and the count of FMAs per division is fixed."""
    for name in ["attn_decode", "attn_prefill", "softmax", "block", "tensor"]:
        text = _disasm(name)
        fmas = len(FLOAT_FMA.findall(text))
        fixups = len(re.findall(r"\bv_div_fixup_f32\b", text))
        assert fixups >= 1
        assert fmas <= 5 * fixups, (name, fmas, fixups)
        assert not re.findall(r"\bv_pk_(fma|mul|add)_f32\b", text)


# ---------------------------------------------------------------- runtime mirror
MATMUL_DECL = """
# declaration of the reference test program's interface (tests/cases/matrix/matmul.hex:2-15)
(def program matmul-2x2-via-mem :
  ([n m k.] {
    (cap.ref mem) (cap.ref mem)
    ({[.n] u64} :) ({[.m] u64} :) ({[.k] u64} :)
    ({({[.n] [.k]} *) u64} :) ({({[.k] [.m]} *) u64} :) ({({[.n] [.m]} *) u64} :)
  })
  -> ([n m k.] (cap.own mem))
  = native)
"""


def test_runtime_parses_and_lists_programs():
    rt = ca.Runtime([MATMUL_DECL])
    names = rt.programs()
    assert "matmul-2x2-via-mem" in names
    assert "nn.softmax" in names and "math.exp-approx" in names
    assert "nn.rmsnorm" in names and "tensor.argmax-f32" in names
    for stdlib in ["tensor.broadcast-f32", "tensor.arange-f32", "tensor.slice-f32",
                   "tensor.concat-f32", "sum-f32", "mean-f32", "max-f32"]:
        assert stdlib in names
    # test programs of the reference (not stdlib) are bound only when declared
    assert "sum-u64" not in names and "dot-u64" not in names
    # identity programs are not declared, so they are not executable
    assert "matmul-right-identity-2x2-via-mem" not in names


def test_runtime_rejects_cuda_dialect_and_bad_source():
    with pytest.raises(ca.ExecError) as e:
        ca.Runtime([], dialect="cuda")
    assert e.value.status == ca.INIT_DIALECT
    with pytest.raises(ca.ExecError) as e:
        ca.Runtime(["(def program x : (f32 val) -> (f32 val) = ("])
    assert e.value.status == ca.INIT_PARSE


def test_runtime_bounds_bracket_nesting():
    """Nesting deeper than the reader's bound is a parse error, not a stack
    overflow."""
    deep = "(" * 100000 + ")" * 100000
    with pytest.raises(ca.ExecError) as e:
        ca.Runtime([deep])
    assert e.value.status == ca.INIT_PARSE
    ok = "(def program nn.softmax : " + "(" * 50 + "cap.own mem" + ")" * 50 + " -> (cap.own mem) = x)"
    ca.Runtime([ok])  # moderate nesting still reads


def test_exec_rejects_null_argument_array():
    """n_args > 0 with a NULL array, or a NULL runtime, is refused before any
    dereference, with a status outside the reference's error kinds."""
    rt = ca.Runtime([MATMUL_DECL])
    L = ca.lib()
    outs = (ca.Value * 1)()
    st = L.catena_runtime_exec(rt._h, b"math.exp-approx", None, 1, outs, 1)
    assert st == ca.EXEC_BAD_CALL
    assert L.catena_runtime_exec(None, b"math.exp-approx", None, 0, outs, 1) == ca.EXEC_BAD_CALL


def test_runtime_signature_mismatch():
    bad = "(def program nn.softmax : (f32 val) -> (cap.own mem) = x)"
    with pytest.raises(ca.ExecError) as e:
        ca.Runtime([bad])
    assert e.value.status == ca.INIT_SIGNATURE_MISMATCH


def test_exec_validation_order():
    """UnknownSourceFunction -> InputArity -> OutputArity -> TypeMismatch,
    as in catena-lang/src/runtime/runtime.rs:180-228; none touches the GPU."""
    rt = ca.Runtime([MATMUL_DECL])
    with pytest.raises(ca.ExecError) as e:
        rt.exec("no-such-program", [], 1)
    assert e.value.status == ca.EXEC_UNKNOWN_SOURCE_FUNCTION
    with pytest.raises(ca.ExecError) as e:
        rt.exec("math.exp-approx", [ca.Value.f32(1.0), ca.Value.f32(2.0)], 1)
    assert (e.value.status, e.value.expected, e.value.actual) == (ca.EXEC_INPUT_ARITY_MISMATCH, 1, 2)
    with pytest.raises(ca.ExecError) as e:
        rt.exec("math.exp-approx", [ca.Value.f32(1.0)], 2)
    assert (e.value.status, e.value.expected, e.value.actual) == (ca.EXEC_OUTPUT_ARITY_MISMATCH, 1, 2)
    # arity is checked before kinds: wrong kind AND wrong output arity -> arity
    with pytest.raises(ca.ExecError) as e:
        rt.exec("math.exp-approx", [ca.Value.u64(1)], 2)
    assert e.value.status == ca.EXEC_OUTPUT_ARITY_MISMATCH
    args = [ca.Value.mem(ca.Mem()), ca.Value.mem(ca.Mem())] + [ca.Value.u64(1)] * 5 + [ca.Value.f32(1.0)]
    with pytest.raises(ca.ExecError) as e:
        rt.exec("matmul-2x2-via-mem", args, 1)
    assert (e.value.status, e.value.index, e.value.expected, e.value.actual) == (
        ca.EXEC_TYPE_MISMATCH, 7, ca.KIND_U64, ca.KIND_F32)
