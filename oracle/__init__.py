"""numpy/ctypes front for the CPU oracle (``oracle/catena_oracle.c``).

TEST INFRASTRUCTURE ONLY.  This package is imported by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``, and
nowhere else: it is the checker for the HIP kernels, never the thing that is
measured or shipped.  The product path (``catena-lang_amd``) does not import
it and fails loudly when its HIP library is missing.

The C restatement follows the reference's generated arithmetic
(catena-lang/src/codegen/ops/reducec.rs:73-130, catena-lang/stdlib/
math.hex:148-199, catena-lang/stdlib/nn.hex:59-122); see the header comment of
catena_oracle.h for which checks pin each function.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_f32p = ctypes.POINTER(ctypes.c_float)


def build() -> str:
    """Compile liboracle.so with the oracle's Makefile (gcc, no-FMA flags)."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.or_f32_bits.argtypes = [ctypes.c_float]
        L.or_f32_bits.restype = ctypes.c_uint32
        L.or_bits_f32.argtypes = [ctypes.c_uint32]
        L.or_bits_f32.restype = ctypes.c_float
        L.or_round_to_u32.argtypes = [ctypes.c_float]
        L.or_round_to_u32.restype = ctypes.c_uint32
        L.or_exp_approx.argtypes = [ctypes.c_float]
        L.or_exp_approx.restype = ctypes.c_float
        L.or_exp_approx_n.argtypes = [_f32p, _f32p, ctypes.c_uint64]
        L.or_exp_approx_n.restype = None
        L.or_exp_approx_nonneg.argtypes = [ctypes.c_float]
        L.or_exp_approx_nonneg.restype = ctypes.c_float
        L.or_f32_to_bf16.argtypes = [ctypes.c_float]
        L.or_f32_to_bf16.restype = ctypes.c_uint16
        L.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_bf16_to_f32.restype = ctypes.c_float
        L.or_fold_sum_f32.argtypes = [_f32p, ctypes.c_uint64]
        L.or_fold_sum_f32.restype = ctypes.c_float
        L.or_fold_max_f32.argtypes = [_f32p, ctypes.c_uint64]
        L.or_fold_max_f32.restype = ctypes.c_float
        L.or_matmul_f32_seq.argtypes = [_f32p, _f32p, _f32p, ctypes.c_uint64,
                                        ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int]
        L.or_matmul_f32_seq.restype = None
        L.or_matmul_bf16_seq.argtypes = [_u16p, _u16p, _f32p, _u16p, ctypes.c_uint64,
                                         ctypes.c_uint64, ctypes.c_uint64, _u64p,
                                         ctypes.c_uint64, ctypes.c_int]
        L.or_matmul_bf16_seq.restype = None
        L.or_softmax_f32.argtypes = [_f32p, _f32p, ctypes.c_uint64]
        L.or_softmax_f32.restype = None
        L.or_attn_decode.argtypes = [_u16p, _u16p, _u16p, _u32p, _f32p, ctypes.c_uint32,
                                     ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                     ctypes.c_float, _u32p, ctypes.c_uint32, ctypes.c_int]
        L.or_attn_decode.restype = None
        for name in ("or_sqrt_newton", "or_sigmoid", "or_silu", "or_sin_approx", "or_cos_approx",
                     "or_sin_full", "or_cos_full"):
            getattr(L, name).argtypes = [ctypes.c_float]
            getattr(L, name).restype = ctypes.c_float
        L.or_map_f32.argtypes = [ctypes.c_int, _f32p, _f32p, ctypes.c_uint64]
        L.or_map_f32.restype = None
        L.or_rmsnorm_f32.argtypes = [_f32p, _f32p, ctypes.c_uint64]
        L.or_rmsnorm_f32.restype = None
        L.or_argmax_f32.argtypes = [_f32p, ctypes.c_uint64]
        L.or_argmax_f32.restype = ctypes.c_uint64
        L.or_rope_inv_freq.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_double]
        L.or_rope_inv_freq.restype = None
        L.or_rope_f32.argtypes = [_f32p, ctypes.c_uint32, _f32p, ctypes.c_uint32]
        L.or_rope_f32.restype = None
        L.or_silu_mul_rows.argtypes = [_f32p, _u16p, ctypes.c_uint64, ctypes.c_uint32,
                                       ctypes.c_uint32]
        L.or_silu_mul_rows.restype = None
        L.or_rope_qkv_rows.argtypes = [_f32p, _f32p, _u32p, _u16p, _u16p, _u16p, ctypes.c_uint64,
                                       ctypes.c_uint32, ctypes.c_uint32]
        L.or_rope_qkv_rows.restype = None
        L.or_rmsnorm_rows.argtypes = [_f32p, _f32p, ctypes.c_uint64, ctypes.c_uint64]
        L.or_rmsnorm_rows.restype = None
        _lib = L
    return _lib


def _p(arr, ptype):
    if arr is None:
        return None
    return arr.ctypes.data_as(ptype)


def default_threads() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0))))


# ---------------------------------------------------------------- scalars
def exp_approx(x: float) -> float:
    return lib().or_exp_approx(float(x))


def exp_approx_vec(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    y = np.empty_like(x)
    lib().or_exp_approx_n(_p(x, _f32p), _p(y, _f32p), x.size)
    return y


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    f = lib().or_f32_to_bf16
    x = np.asarray(x, np.float32)
    return np.array([f(float(v)) for v in x.ravel()], np.uint16).reshape(x.shape)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    """Exact widening (bit shift), same as or_bf16_to_f32."""
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits_np(x: np.ndarray) -> np.ndarray:
    """Vectorised RNE float32 -> bf16 bits, identical rule to or_f32_to_bf16."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


# ---------------------------------------------------------------- folds
def fold_sum_f32(x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, np.float32)
    return lib().or_fold_sum_f32(_p(x, _f32p), x.size)


def fold_max_f32(x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, np.float32)
    return lib().or_fold_max_f32(_p(x, _f32p), x.size)


def softmax_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().or_softmax_f32(_p(x, _f32p), _p(y, _f32p), x.size)
    return y


# ---------------------------------------------------------------- matmul
def matmul_f32(a: np.ndarray, b: np.ndarray, threads: int | None = None) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    n, k = a.shape
    k2, m = b.shape
    assert k == k2
    c = np.empty((n, m), np.float32)
    lib().or_matmul_f32_seq(_p(a, _f32p), _p(b, _f32p), _p(c, _f32p), n, m, k,
                            threads or default_threads())
    return c


def matmul_bf16(a_bits: np.ndarray, b_bits: np.ndarray, rows=None,
                threads: int | None = None):
    """Returns (c32, c16) for all rows or for the listed rows."""
    a = np.ascontiguousarray(a_bits, np.uint16)
    b = np.ascontiguousarray(b_bits, np.uint16)
    n, k = a.shape
    k2, m = b.shape
    assert k == k2
    rows_arr = None if rows is None else np.ascontiguousarray(rows, np.uint64)
    nr = n if rows_arr is None else rows_arr.size
    c32 = np.empty((nr, m), np.float32)
    c16 = np.empty((nr, m), np.uint16)
    lib().or_matmul_bf16_seq(_p(a, _u16p), _p(b, _u16p), _p(c32, _f32p), _p(c16, _u16p),
                             n, m, k, _p(rows_arr, _u64p), nr, threads or default_threads())
    return c32, c16


# ---------------------------------------------------------------- attention
def attn_decode(q, k, v, lens, scale: float, heads=None, threads: int | None = None):
    """q [B,H,D], k/v [B,H,L,D] bf16 bits, lens [B] -> o [B,H,D] (or [n,D])."""
    q = np.ascontiguousarray(q, np.uint16)
    k = np.ascontiguousarray(k, np.uint16)
    v = np.ascontiguousarray(v, np.uint16)
    lens = np.ascontiguousarray(lens, np.uint32)
    B, H, L, D = k.shape
    assert q.shape == (B, H, D) and v.shape == k.shape and lens.shape == (B,)
    assert int(lens.max(initial=0)) <= L
    hl = None if heads is None else np.ascontiguousarray(heads, np.uint32)
    o = np.empty((B, H, D) if hl is None else (hl.size, D), np.float32)
    lib().or_attn_decode(_p(q, _u16p), _p(k, _u16p), _p(v, _u16p), _p(lens, _u32p),
                         _p(o, _f32p), B, H, L, D, float(scale), _p(hl, _u32p),
                         0 if hl is None else hl.size, threads or default_threads())
    return o


# ---------------------------------------------------------------- decoder-block pieces
def scalar(name: str, x: float) -> float:
    return getattr(lib(), "or_" + name)(float(x))


def scalar_vec(name: str, x: np.ndarray) -> np.ndarray:
    f = getattr(lib(), "or_" + name)
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()], np.float32)


MAP_OPS = {"exp_approx": 0, "sqrt_newton": 1, "sigmoid": 2, "silu": 3, "sin_approx": 4,
           "cos_approx": 5, "sin_full": 6}


def map_f32(name: str, x: np.ndarray) -> np.ndarray:
    """A scalar program over an array (or_map_f32; name as in MAP_OPS)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    y = np.empty_like(x)
    lib().or_map_f32(MAP_OPS[name], _p(x, _f32p), _p(y, _f32p), x.size)
    return y


def rmsnorm_f32(x: np.ndarray) -> np.ndarray:
    """nn.rmsnorm per row of a 1-D or 2-D array."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    n = x.shape[-1]
    lib().or_rmsnorm_rows(_p(x, _f32p), _p(y, _f32p), x.size // n if n else 0, n)
    return y


def argmax_f32(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, np.float32)
    return int(lib().or_argmax_f32(_p(x, _f32p), x.size))


def rope_inv_freq(d: int, base: float) -> np.ndarray:
    out = np.empty(d // 2, np.float32)
    lib().or_rope_inv_freq(_p(out, _f32p), d, float(base))
    return out


def rope_f32(x: np.ndarray, pos: int, inv_freq: np.ndarray) -> np.ndarray:
    """Rotate one head vector (copy)."""
    y = np.ascontiguousarray(x, np.float32).copy()
    f = np.ascontiguousarray(inv_freq, np.float32)
    lib().or_rope_f32(_p(y, _f32p), int(pos), _p(f, _f32p), y.size)
    return y
