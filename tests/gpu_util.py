"""Helpers shared by the GPU parity tests (not collected by pytest)."""
import sys

import numpy as np

import catena_amd as ca
import oracle

U = 2.0 ** -24  # f32 unit roundoff


def say(msg: str) -> None:
    """Name the case before each GPU step so a failing run shows where it was."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def dev_normal_bf16(n: int, seed: int, stream: int, scale: float = 1.0):
    buf = ca.Buffer(n * 2)
    ca.fill_normal_bf16(buf, n, seed, stream, scale)
    return buf


def bf16_order(bits: np.ndarray) -> np.ndarray:
    """Map bf16 bit patterns to integers whose differences count ULPs."""
    b = bits.astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)


def bf16_ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return np.abs(bf16_order(a) - bf16_order(b))


def bf16_ulp_of(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |x| (8 significand bits)."""
    ax = np.maximum(np.abs(x.astype(np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(ax)) - 7)


def hash_bits(arr: np.ndarray) -> int:
    import hashlib
    return int(hashlib.sha256(np.ascontiguousarray(arr).tobytes()).hexdigest()[:16], 16)


def as_f32(bits16: np.ndarray) -> np.ndarray:
    return oracle.bf16_bits_to_f32(bits16)


def gemm_within_bound(a16: np.ndarray, b16: np.ndarray, got32: np.ndarray) -> float:
    """Assert the MFMA-order f32 GEMM bound |C - AB| <= 8 (K/32 + 1) u sum|A||B|
    (A, B bf16 bits, C exact in float64); returns the worst ratio to the bound."""
    af = as_f32(a16).astype(np.float64)
    bf = as_f32(b16).astype(np.float64)
    k = a16.shape[1]
    bound = 8 * (k / 32 + 1) * U * (np.abs(af) @ np.abs(bf))
    err = np.abs(got32.astype(np.float64) - af @ bf)
    ratio = float((err / np.maximum(bound, 1e-300)).max())
    assert np.all(err <= bound), ratio
    return ratio
