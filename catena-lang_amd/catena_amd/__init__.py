"""ctypes binding of libcatena_mi355x (include/catena_mi355x.h).

This is plumbing for Python callers (tests, bench, smoke): every call goes
through the C ABI into the native library and its gfx950 kernels.  There is
no Python or CPU fallback; if the library or its code objects are missing,
`lib()` raises.

Layout mirrors the C header:
  * device/pool:   init, Buffer (catena_mem_t), synchronize, stream
  * kernel ABI:    gemm_f32_exact, gemm_bf16, attn_decode_bf16, softmax_f32, ...
                   and the decoder-block pieces (rmsnorm, rope, silu_mul, argmax, ...)
  * decoder:       Decoder (catena_mi355x_decoder_*)
  * program ABI:   program_* functions (fail-stop: they trap on bad input)
  * runtime:       Runtime (catena_runtime_*), mirrors Runtime::from_sources /
                   exec / mem_* of catena-lang/src/runtime/runtime.rs:104-247
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.dirname(_HERE)
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libcatena_mi355x.so")

CATENA_OK = 0
STATUS_NAMES = {0: "OK", 1: "INVALID_ARGUMENT", 2: "UNSUPPORTED", 3: "HIP", 4: "OUT_OF_MEMORY",
                5: "NOT_INITIALIZED", 6: "LOAD"}

# catena_value_kind_t (ValueKind, catena-lang/src/runtime/value.rs:15-21)
KIND_BOOL, KIND_U32, KIND_U64, KIND_F32, KIND_MEM = range(5)
KIND_NAMES = {0: "Bool", 1: "U32", 2: "U64", 3: "F32", 4: "Mem"}

EXEC_OK = 0
EXEC_UNKNOWN_SOURCE_FUNCTION = 1
EXEC_INPUT_ARITY_MISMATCH = 2
EXEC_OUTPUT_ARITY_MISMATCH = 3
EXEC_TYPE_MISMATCH = 4
INIT_PARSE = 10
INIT_NO_LOWERING = 11
INIT_SIGNATURE_MISMATCH = 12
INIT_DIALECT = 13
INIT_DEVICE = 14
INIT_HOST_MEMORY = 15
EXEC_BAD_CALL = 20


class CatenaError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[{STATUS_NAMES.get(status, status)}] {message}")
        self.status = status


class Mem(ctypes.Structure):
    """catena_mem_t: {void* data; uint64_t len} (bytes)."""
    _fields_ = [("data", ctypes.c_void_p), ("len", ctypes.c_uint64)]


class _ValueUnion(ctypes.Union):
    _fields_ = [("b", ctypes.c_uint8), ("u32", ctypes.c_uint32), ("u64", ctypes.c_uint64),
                ("f32", ctypes.c_float), ("mem", Mem)]


class Value(ctypes.Structure):
    """catena_value_t: tagged Value (catena-lang/src/runtime/value.rs:5-12)."""
    _fields_ = [("kind", ctypes.c_int), ("as_", _ValueUnion)]

    @staticmethod
    def bool(v: bool) -> "Value":
        x = Value(); x.kind = KIND_BOOL; x.as_.b = 1 if v else 0; return x

    @staticmethod
    def u32(v: int) -> "Value":
        x = Value(); x.kind = KIND_U32; x.as_.u32 = v; return x

    @staticmethod
    def u64(v: int) -> "Value":
        x = Value(); x.kind = KIND_U64; x.as_.u64 = v; return x

    @staticmethod
    def f32(v: float) -> "Value":
        x = Value(); x.kind = KIND_F32; x.as_.f32 = v; return x

    @staticmethod
    def mem(m: Mem) -> "Value":
        x = Value(); x.kind = KIND_MEM; x.as_.mem = m; return x

    def get(self):
        k = self.kind
        if k == KIND_BOOL:
            return self.as_.b
        if k == KIND_U32:
            return self.as_.u32
        if k == KIND_U64:
            return self.as_.u64
        if k == KIND_F32:
            return self.as_.f32
        return self.as_.mem


_lib = None
_vp = ctypes.c_void_p
_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_f32 = ctypes.c_float
_int = ctypes.c_int

# name -> (restype, argtypes); the list is the header's full export surface.
SIGNATURES = {
    "catena_mi355x_init": (_int, [_int]),
    "catena_mi355x_shutdown": (_int, []),
    "catena_mi355x_last_error": (ctypes.c_char_p, []),
    "catena_mi355x_stream": (_vp, []),
    "catena_mi355x_synchronize": (_int, []),
    "catena_mem_alloc": (_int, [_u64, ctypes.POINTER(Mem)]),
    "catena_mem_free": (_int, [ctypes.POINTER(Mem)]),
    "catena_mem_write": (_int, [Mem, _u64, _vp, _u64]),
    "catena_mem_read": (_int, [Mem, _u64, _vp, _u64]),
    "catena_pool_stats": (_int, [ctypes.POINTER(_u64)] * 3),
    "catena_pool_trim": (_int, []),
    "catena_mi355x_gemm_f32_exact": (_int, [_vp, _vp, _vp, _u64, _u64, _u64]),
    "catena_mi355x_gemm_bf16": (_int, [_vp, _vp, _vp, _u64, _u64, _u64, _int]),
    "catena_mi355x_gemm_bf16_argmax": (_int, [_vp, _vp, _vp, _vp, _u64, _u64, _u64]),
    "catena_mi355x_gemm_bf16_decode_plan": (_int, [_u64, _u64, _u64, ctypes.POINTER(_u32),
                                                   ctypes.POINTER(_u64)]),
    "catena_mi355x_gemm_bf16_decode_noalloc": (_int, [_vp, _vp, _vp, _u64, _u64, _u64, _int]),
    "catena_mi355x_attn_decode_bf16": (_int, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _f32]),
    "catena_mi355x_softmax_f32": (_int, [_vp, _vp, _u64, _u64]),
    "catena_mi355x_exp_approx_f32": (_int, [_vp, _vp, _u64]),
    "catena_mi355x_map_f32": (_int, [_u32, _vp, _vp, _u64]),
    "catena_mi355x_fill_normal_bf16": (_int, [_vp, _u64, _u64, _u64, _f32]),
    "catena_mi355x_fill_uniform_f32": (_int, [_vp, _u64, _u64, _u64]),
    "catena_mi355x_copy_bytes": (_int, [_vp, _vp, _u64]),
    "catena_mi355x_attn_causal_bf16": (_int, [_vp] * 5 + [_u32] * 5 + [_f32, _int]),
    "catena_mi355x_rmsnorm_f32": (_int, [_vp, _vp, _u64, _u64]),
    "catena_mi355x_residual_rmsnorm_bf16": (_int, [_vp] * 5 + [_u64, _u64]),
    "catena_mi355x_embed_bf16": (_int, [_vp, _vp, _vp, _u64, _u32, _u32]),
    "catena_mi355x_rope_inv_freq": (_int, [ctypes.POINTER(_f32), _u32, ctypes.c_double]),
    "catena_mi355x_rope_qkv_bf16": (_int, [_vp] * 6 + [_u32] * 5),
    "catena_mi355x_silu_mul_bf16": (_int, [_vp, _vp, _u64, _u32, _u32]),
    "catena_mi355x_gemm_bf16_silu": (_int, [_vp, _vp, _vp, _u64, _u64, _u64]),
    "catena_mi355x_rope_table_f32": (_int, [_vp, _vp, _u32, _u32]),
    "catena_mi355x_gemm_bf16_rope_qkv": (_int, [_vp] * 7 + [_u32] * 4 + [_u64]),
    "catena_mi355x_gemm_bf16_ksplit_f32": (_int, [_vp, _vp, _vp, _u64, _u64, _u64, _u32]),
    "catena_mi355x_argmax_f32": (_int, [_vp, _vp, _u64, _u64]),
    "catena_mi355x_broadcast_f32": (_int, [_vp, _u64, _f32]),
    "catena_mi355x_arange_f32": (_int, [_vp, _u64]),
    "catena_mi355x_copy_f32": (_int, [_vp, _vp, _u64]),
    "catena_mi355x_sum_f32": (_int, [_vp, _vp, _u64, _u64]),
    "catena_mi355x_mean_f32": (_int, [_vp, _vp, _u64, _u64]),
    "catena_mi355x_max_f32": (_int, [_vp, _vp, _u64, _u64]),
    "catena_mi355x_sum_u64": (_int, [_vp, _vp, _u64, _u64]),
    "catena_mi355x_dot_u64": (_int, [_vp, _vp, _vp, _u64, _u64]),
    "program_tensor_broadcast_f32": (None, [_f32, _u64, ctypes.POINTER(Mem)]),
    "program_tensor_arange_f32": (None, [_u64, ctypes.POINTER(Mem)]),
    "program_tensor_slice_f32": (None, [Mem, _u64, _u64, ctypes.POINTER(Mem)]),
    "program_tensor_concat_f32": (None, [Mem, Mem, ctypes.POINTER(Mem)]),
    "program_sum_f32": (None, [Mem, ctypes.POINTER(_f32)]),
    "program_mean_f32": (None, [Mem, ctypes.POINTER(_f32)]),
    "program_max_f32": (None, [Mem, ctypes.POINTER(_f32)]),
    "program_sum_u64": (None, [Mem, ctypes.POINTER(_u64)]),
    "program_dot_u64": (None, [Mem, Mem, ctypes.POINTER(_u64)]),
    "program_nn_rmsnorm": (None, [Mem, ctypes.POINTER(Mem)]),
    "program_tensor_argmax_f32": (None, [Mem, ctypes.POINTER(_u64)]),
    "catena_mi355x_decoder_create": (_int, [_vp, ctypes.POINTER(_vp)]),
    "catena_mi355x_decoder_destroy": (None, [_vp]),
    "catena_mi355x_decoder_tensor": (_int, [_vp, _u32, _u32, ctypes.POINTER(Mem)]),
    "catena_mi355x_decoder_init_weights": (_int, [_vp, _u64, _f32]),
    "catena_mi355x_decoder_prefill": (_int, [_vp, _vp, _u32, _u32, _vp]),
    "catena_mi355x_decoder_generate": (_int, [_vp, _u32, _vp]),
    "program_matmul_2x2_via_mem": (None, [Mem, Mem] + [_u64] * 6 + [ctypes.POINTER(Mem)]),
    "program_matmul_right_identity_2x2_via_mem": (None, [Mem, _u64, _u64, ctypes.POINTER(Mem)]),
    "program_matmul_left_identity_2x2_via_mem": (None, [Mem, _u64, _u64, ctypes.POINTER(Mem)]),
    "program_nn_softmax": (None, [Mem, ctypes.POINTER(Mem)]),
    "program_math_exp_approx": (None, [_f32, ctypes.POINTER(_f32)]),
    "program_math_sqrt": (None, [_f32, ctypes.POINTER(_f32)]),
    "program_nn_sigmoid": (None, [_f32, ctypes.POINTER(_f32)]),
    "program_nn_silu": (None, [_f32, ctypes.POINTER(_f32)]),
    "program_math_sin_approx": (None, [_f32, ctypes.POINTER(_f32)]),
    "program_math_cos_approx": (None, [_f32, ctypes.POINTER(_f32)]),
    "program_math_sin_approx_full": (None, [_f32, ctypes.POINTER(_f32)]),
    "program_bf16_matmul_via_mem": (None, [Mem, Mem] + [_u64] * 6 + [ctypes.POINTER(Mem)]),
    "program_attn_decode_via_mem": (None, [Mem, Mem, Mem, Mem] + [_u64] * 4 + [_f32, ctypes.POINTER(Mem)]),
    "catena_runtime_from_sources": (_int, [ctypes.POINTER(ctypes.c_char_p), ctypes.c_size_t,
                                           ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "catena_runtime_destroy": (None, [_vp]),
    "catena_runtime_exec": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(Value), ctypes.c_size_t,
                                   ctypes.POINTER(Value), ctypes.c_size_t]),
    "catena_runtime_last_error_detail": (_int, [ctypes.POINTER(ctypes.c_int64)] * 3),
    "catena_runtime_program_count": (ctypes.c_size_t, [_vp]),
    "catena_runtime_program_name": (ctypes.c_char_p, [_vp, ctypes.c_size_t]),
    "catena_runtime_mem_u64": (_int, [_vp, ctypes.POINTER(_u64), ctypes.c_size_t, ctypes.POINTER(Value)]),
    "catena_runtime_mem_f32": (_int, [_vp, ctypes.POINTER(_f32), ctypes.c_size_t, ctypes.POINTER(Value)]),
}


def lib():
    """Load libcatena_mi355x.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run `python catena-lang_amd/build.py` "
                               "(or __graft_entry__.build()) first")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return (lib().catena_mi355x_last_error() or b"").decode()


def check(status: int) -> None:
    if status != CATENA_OK:
        raise CatenaError(status, last_error())


_atexit_registered = False


def init(device: int = 0) -> None:
    """Initialise the library on `device`; an orderly shutdown is registered
    to run at interpreter exit (before the HIP runtime's own teardown)."""
    global _atexit_registered
    check(lib().catena_mi355x_init(device))
    if not _atexit_registered:
        import atexit
        atexit.register(shutdown)
        _atexit_registered = True


def shutdown() -> None:
    """catena_mi355x_shutdown: wait for the library stream, release the
    library's own device memory, unload its code objects, destroy the
    stream."""
    if _lib is not None:
        check(_lib.catena_mi355x_shutdown())


def synchronize() -> None:
    check(lib().catena_mi355x_synchronize())


def stream() -> int:
    s = lib().catena_mi355x_stream()
    if not s:
        raise CatenaError(5, last_error())
    return s


def pool_stats():
    a, b, c = _u64(), _u64(), _u64()
    check(lib().catena_pool_stats(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)))
    return {"bytes_live": a.value, "bytes_cached": b.value, "device_allocs": c.value}


class Buffer:
    """Owning handle of a pool buffer (catena_mem_t); freed on close/GC."""

    def __init__(self, nbytes: int = 0, mem: Mem | None = None):
        if mem is not None:
            self.mem = mem
        else:
            self.mem = Mem()
            check(lib().catena_mem_alloc(int(nbytes), ctypes.byref(self.mem)))

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "Buffer":
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes)
        b.write(arr)
        return b

    @property
    def ptr(self) -> int:
        return self.mem.data or 0

    @property
    def nbytes(self) -> int:
        return self.mem.len

    def write(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        check(lib().catena_mem_write(self.mem, offset, arr.ctypes.data_as(_vp), arr.nbytes))

    def read(self, dtype, shape=None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = (self.mem.len - offset) // dtype.itemsize if shape is None else int(np.prod(shape))
        out = np.empty(count, dtype)
        check(lib().catena_mem_read(self.mem, offset, out.ctypes.data_as(_vp), out.nbytes))
        return out if shape is None else out.reshape(shape)

    def close(self) -> None:
        if getattr(self, "mem", None) is not None and self.mem.data and _lib is not None:
            check(_lib.catena_mem_free(ctypes.byref(self.mem)))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------------------ kernel ABI
def _p(x) -> int:
    return x.ptr if isinstance(x, Buffer) else int(x)


def gemm_f32_exact(a, b, c, n: int, m: int, k: int) -> None:
    check(lib().catena_mi355x_gemm_f32_exact(_p(a), _p(b), _p(c), n, m, k))


def gemm_bf16(a, b, c, n: int, m: int, k: int, out_f32: bool = False) -> None:
    check(lib().catena_mi355x_gemm_bf16(_p(a), _p(b), _p(c), n, m, k, 1 if out_f32 else 0))


def gemm_bf16_argmax(a, b, c, idx, n: int, m: int, k: int) -> None:
    """LM head: c = a * b (f32, decode shape) and idx[r] = tensor.argmax-f32
    of row r of c, in one launch."""
    check(lib().catena_mi355x_gemm_bf16_argmax(_p(a), _p(b), _p(c), _p(idx), n, m, k))


def gemm_bf16_decode_noalloc(a, b, c, n: int, m: int, k: int, out_f32: bool = False) -> None:
    """Allocation-free decode-shape GEMM (partials in the library's fixed
    device scratch)."""
    check(lib().catena_mi355x_gemm_bf16_decode_noalloc(_p(a), _p(b), _p(c), n, m, k,
                                                       1 if out_f32 else 0))


def gemm_bf16_decode_plan(n: int, m: int, k: int):
    """(k groups, partials bytes) of the decode-shape GEMM for this shape;
    needs no device."""
    groups, nbytes = _u32(), _u64()
    check(lib().catena_mi355x_gemm_bf16_decode_plan(n, m, k, ctypes.byref(groups),
                                                    ctypes.byref(nbytes)))
    return groups.value, nbytes.value


def attn_decode_bf16(q, k, v, lens, o, batch: int, heads: int, max_len: int, head_dim: int,
                     scale: float) -> None:
    check(lib().catena_mi355x_attn_decode_bf16(_p(q), _p(k), _p(v), _p(lens), _p(o), batch, heads,
                                               max_len, head_dim, scale))


def softmax_f32(x, y, rows: int, n: int) -> None:
    check(lib().catena_mi355x_softmax_f32(_p(x), _p(y), rows, n))


def exp_approx_f32(x, y, n: int) -> None:
    check(lib().catena_mi355x_exp_approx_f32(_p(x), _p(y), n))


# catena_map_op_t
(MAP_EXP_APPROX, MAP_SQRT, MAP_SIGMOID, MAP_SILU, MAP_SIN_APPROX, MAP_COS_APPROX,
 MAP_SIN_APPROX_FULL) = range(7)


def map_f32(op: int, x, y, n: int) -> None:
    """A scalar stdlib program elementwise (catena_mi355x_map_f32)."""
    check(lib().catena_mi355x_map_f32(op, _p(x), _p(y), n))


def fill_normal_bf16(out, n: int, seed: int, stream_id: int, scale: float = 1.0) -> None:
    check(lib().catena_mi355x_fill_normal_bf16(_p(out), n, seed, stream_id, scale))


def fill_uniform_f32(out, n: int, seed: int, stream_id: int) -> None:
    check(lib().catena_mi355x_fill_uniform_f32(_p(out), n, seed, stream_id))


def copy_bytes(dst, src, n: int) -> None:
    check(lib().catena_mi355x_copy_bytes(_p(dst), _p(src), n))


def attn_causal_bf16(q, k, v, lens, o, batch: int, tq: int, heads: int, max_len: int,
                     head_dim: int, scale: float, out_f32: bool = False) -> None:
    check(lib().catena_mi355x_attn_causal_bf16(_p(q), _p(k), _p(v), _p(lens), _p(o), batch, tq,
                                               heads, max_len, head_dim, scale,
                                               1 if out_f32 else 0))


def rmsnorm_f32(x, y, rows: int, n: int) -> None:
    check(lib().catena_mi355x_rmsnorm_f32(_p(x), _p(y), rows, n))


def residual_rmsnorm_bf16(x, resid, row_index, h_out, y, rows: int, n: int) -> None:
    opt = lambda b: None if b is None else _p(b)  # noqa: E731
    check(lib().catena_mi355x_residual_rmsnorm_bf16(_p(x), opt(resid), opt(row_index), opt(h_out),
                                                    _p(y), rows, n))


def embed_bf16(tokens, table, x, rows: int, vocab: int, d: int) -> None:
    check(lib().catena_mi355x_embed_bf16(_p(tokens), _p(table), _p(x), rows, vocab, d))


def rope_inv_freq(head_dim: int, base: float) -> np.ndarray:
    out = np.empty(head_dim // 2, np.float32)
    check(lib().catena_mi355x_rope_inv_freq(out.ctypes.data_as(ctypes.POINTER(_f32)), head_dim,
                                            float(base)))
    return out


def rope_qkv_bf16(qkv, inv_freq, lens, q, k_cache, v_cache, batch: int, tq: int, heads: int,
                  head_dim: int, max_len: int) -> None:
    check(lib().catena_mi355x_rope_qkv_bf16(_p(qkv), _p(inv_freq), _p(lens), _p(q), _p(k_cache),
                                            _p(v_cache), batch, tq, heads, head_dim, max_len))


def silu_mul_bf16(gu, out, rows: int, ffn: int, group: int = 0) -> None:
    check(lib().catena_mi355x_silu_mul_bf16(_p(gu), _p(out), rows, ffn, group))


def gemm_bf16_silu(a, b, act, n: int, m: int, k: int) -> None:
    """act[n][m/2] = bf16(silu(gate) * up) of A[n][k] x B[k][m] (gate / up in
    groups of 64 columns), the GEMM and catena_mi355x_silu_mul_bf16 in one."""
    check(lib().catena_mi355x_gemm_bf16_silu(_p(a), _p(b), _p(act), n, m, k))


def rope_table_f32(inv_freq, tab, positions: int, head_dim: int) -> None:
    """tab[pos][i] = (cos, sin) of (f32)pos * inv_freq[i], i < head_dim / 2."""
    check(lib().catena_mi355x_rope_table_f32(_p(inv_freq), _p(tab), positions, head_dim))


def gemm_bf16_rope_qkv(a, w, rope_tab, lens, q, k_cache, v_cache, batch: int, tq: int, heads: int,
                       max_len: int, k: int) -> None:
    """The q / k / v projection of a[batch*tq][k] by w[k][3*heads*128] with
    RoPE and the cache append fused (gemm_bf16 f32 then rope_qkv_bf16)."""
    check(lib().catena_mi355x_gemm_bf16_rope_qkv(_p(a), _p(w), _p(rope_tab), _p(lens), _p(q),
                                                 _p(k_cache), _p(v_cache), batch, tq, heads,
                                                 max_len, k))


def gemm_bf16_ksplit_f32(a, b, parts, n: int, m: int, k: int, splits: int) -> None:
    """parts[z][n][m] = A[:, kz] x B[kz, :] over the z-th of `splits` equal k ranges."""
    check(lib().catena_mi355x_gemm_bf16_ksplit_f32(_p(a), _p(b), _p(parts), n, m, k, splits))


def argmax_f32(x, idx, rows: int, n: int) -> None:
    check(lib().catena_mi355x_argmax_f32(_p(x), _p(idx), rows, n))


def broadcast_f32(out, n: int, value: float) -> None:
    check(lib().catena_mi355x_broadcast_f32(_p(out), n, value))


def arange_f32(out, n: int) -> None:
    check(lib().catena_mi355x_arange_f32(_p(out), n))


def copy_f32(dst, src, n: int) -> None:
    check(lib().catena_mi355x_copy_f32(_p(dst), _p(src), n))


def sum_f32(x, out, rows: int, n: int) -> None:
    check(lib().catena_mi355x_sum_f32(_p(x), _p(out), rows, n))


def mean_f32(x, out, rows: int, n: int) -> None:
    check(lib().catena_mi355x_mean_f32(_p(x), _p(out), rows, n))


def max_f32(x, out, rows: int, n: int) -> None:
    check(lib().catena_mi355x_max_f32(_p(x), _p(out), rows, n))


def sum_u64(x, out, rows: int, n: int) -> None:
    check(lib().catena_mi355x_sum_u64(_p(x), _p(out), rows, n))


def dot_u64(a, b, out, rows: int, n: int) -> None:
    check(lib().catena_mi355x_dot_u64(_p(a), _p(b), _p(out), rows, n))


# ------------------------------------------------------------------ decoder
class DecoderConfig(ctypes.Structure):
    """catena_decoder_config_t."""
    _fields_ = [("d_model", _u32), ("n_heads", _u32), ("head_dim", _u32), ("ffn_dim", _u32),
                ("n_layers", _u32), ("vocab", _u32), ("max_batch", _u32), ("max_len", _u32),
                ("rope_base", _f32)]


# catena_decoder_tensor_t
(DEC_EMBED, DEC_W_QKV, DEC_W_O, DEC_W_GU, DEC_W_DOWN, DEC_W_LM, DEC_K_CACHE, DEC_V_CACHE,
 DEC_INV_FREQ, DEC_X, DEC_XN, DEC_QKV, DEC_Q, DEC_ATTN, DEC_ATTN_PROJ, DEC_H, DEC_HN, DEC_GU,
 DEC_ACT, DEC_FFN_OUT, DEC_FINAL_H, DEC_FINAL_XN, DEC_LOGITS, DEC_LENS, DEC_EMBED_NORM) = range(25)


class Decoder:
    """Handle of a catena_decoder_t (device-resident weights, caches and
    activations; prefill / generate enqueue on the library stream)."""

    def __init__(self, d_model: int, n_heads: int, ffn_dim: int, n_layers: int, vocab: int,
                 max_batch: int, max_len: int, head_dim: int = 128, rope_base: float = 10000.0):
        self.cfg = DecoderConfig(d_model, n_heads, head_dim, ffn_dim, n_layers, vocab, max_batch,
                                 max_len, rope_base)
        h = _vp()
        check(lib().catena_mi355x_decoder_create(ctypes.byref(self.cfg), ctypes.byref(h)))
        self._h = h

    def tensor(self, which: int, layer: int = 0) -> Mem:
        m = Mem()
        check(lib().catena_mi355x_decoder_tensor(self._h, which, layer, ctypes.byref(m)))
        return m

    def read(self, which: int, dtype, layer: int = 0) -> np.ndarray:
        return mem_to_array(self.tensor(which, layer), dtype)

    def init_weights(self, seed: int, std: float = 0.02) -> None:
        check(lib().catena_mi355x_decoder_init_weights(self._h, seed, std))

    def prefill(self, tokens, batch: int, t: int, next_tokens) -> None:
        check(lib().catena_mi355x_decoder_prefill(self._h, _p(tokens), batch, t, _p(next_tokens)))

    def generate(self, steps: int, out) -> None:
        check(lib().catena_mi355x_decoder_generate(self._h, steps, _p(out)))

    def close(self):
        if getattr(self, "_h", None):
            lib().catena_mi355x_decoder_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------------------ runtime
class ExecError(RuntimeError):
    def __init__(self, status: int, message: str, index: int, expected: int, actual: int):
        super().__init__(message)
        self.status, self.index, self.expected, self.actual = status, index, expected, actual


class Runtime:
    """Mirror of catena's Runtime (catena-lang/src/runtime/runtime.rs:24-247)."""

    def __init__(self, sources=(), dialect: str = "hip"):
        L = lib()
        enc = [s.encode() for s in sources]
        arr = (ctypes.c_char_p * max(1, len(enc)))(*enc)
        h = _vp()
        st = L.catena_runtime_from_sources(arr, len(enc), dialect.encode(), ctypes.byref(h))
        if st != 0:
            raise ExecError(st, last_error(), -1, -1, -1)
        self._h = h

    def programs(self) -> list[str]:
        L = lib()
        return [L.catena_runtime_program_name(self._h, i).decode()
                for i in range(L.catena_runtime_program_count(self._h))]

    def mem_f32(self, values) -> Value:
        a = np.ascontiguousarray(values, np.float32)
        v = Value()
        check(lib().catena_runtime_mem_f32(self._h, a.ctypes.data_as(ctypes.POINTER(_f32)), a.size,
                                           ctypes.byref(v)))
        return v

    def mem_u64(self, values) -> Value:
        a = np.ascontiguousarray(values, np.uint64)
        v = Value()
        check(lib().catena_runtime_mem_u64(self._h, a.ctypes.data_as(ctypes.POINTER(_u64)), a.size,
                                           ctypes.byref(v)))
        return v

    def exec(self, name: str, args, n_outputs: int) -> list[Value]:
        L = lib()
        ins = (Value * max(1, len(args)))(*args)
        outs = (Value * max(1, n_outputs))()
        st = L.catena_runtime_exec(self._h, name.encode(), ins, len(args), outs, n_outputs)
        if st != 0:
            i, e, a = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
            L.catena_runtime_last_error_detail(ctypes.byref(i), ctypes.byref(e), ctypes.byref(a))
            raise ExecError(st, last_error(), i.value, e.value, a.value)
        return list(outs)[:n_outputs]

    def close(self):
        if getattr(self, "_h", None):
            lib().catena_runtime_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def mem_to_array(m: Mem, dtype) -> np.ndarray:
    """Host copy of a runtime Mem (Mem::to_f32_vec / to_u64_vec,
    catena-lang/src/runtime/mem.rs:44-70): asserts len % itemsize == 0."""
    dtype = np.dtype(dtype)
    assert m.len % dtype.itemsize == 0
    out = np.empty(m.len // dtype.itemsize, dtype)
    check(lib().catena_mem_read(m, 0, out.ctypes.data_as(_vp), out.nbytes))
    return out


def mem_write(m: Mem, arr: np.ndarray, offset: int = 0) -> None:
    """Host -> device copy into a runtime Mem (catena_mem_write)."""
    arr = np.ascontiguousarray(arr)
    check(lib().catena_mem_write(m, offset, arr.ctypes.data_as(_vp), arr.nbytes))


def mem_free(m: Mem) -> None:
    check(lib().catena_mem_free(ctypes.byref(m)))
