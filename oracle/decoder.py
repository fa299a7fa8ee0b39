"""CPU oracle of the decoder built on the library's kernels (composition of
the restated stdlib pieces in catena_oracle.c / catena_oracle_block.c).

TEST INFRASTRUCTURE ONLY (imported by tests/, smoke() and bench.py's
cpu_baseline leg).  Each stage takes numpy arrays (bf16 as uint16 bits) and
returns what the corresponding GPU stage must produce: bitwise for the
elementwise / fold stages, and the sequential-order reference value for the
GEMMs (whose GPU order is MFMA's, checked under a bound).

Stage definitions (one IEEE op per node, operands in this order):
  residual_rmsnorm_bf16: h = x + r;  y = bf16(nn.rmsnorm(h))
                         (catena-lang/stdlib/nn.hex:154-182)
  rope_qkv:              pairs (i, i + D/2) of each q / k head rotate by
                         theta = f32(pos) * inv_freq[i]:
                         y1 = x1*c - x2*s, y2 = x2*c + x1*s with
                         s = math.sin-approx-full(theta)
                         (catena-lang/stdlib/math.hex:52-103) and c the same
                         reduction with the quadrant advanced by one
  attn_causal:           query tq of sequence b = decode attention over the
                         first lens[b] - (Tq - 1 - tq) cache rows
  silu_mul_bf16:         bf16(nn.silu(g) * u)   (catena-lang/stdlib/nn.hex:1-21);
                         the decoder's W_gu interleaves gate / up by 64 columns
  argmax:                tensor.argmax-f32 (catena-lang/stdlib/tensor.hex:204-227)
"""
from __future__ import annotations

import numpy as np

import ctypes

from . import (argmax_f32, attn_decode, bf16_bits_to_f32, f32_to_bf16_bits_np, lib,
               matmul_bf16, rmsnorm_f32, rope_f32)


def _ptr(arr, ctype):
    return arr.ctypes.data_as(ctypes.POINTER(ctype))


def residual_rmsnorm_bf16(x, r=None):
    """-> (h f32, y bf16 bits) per row."""
    x = np.asarray(x, np.float32)
    h = x if r is None else (x + np.asarray(r, np.float32)).astype(np.float32)
    return h, f32_to_bf16_bits_np(rmsnorm_f32(h))


def silu_mul_bf16(gu, ffn: int, group: int = 0):
    """group = 0: columns gate | up; group = G: interleaved in groups of G."""
    gu = np.ascontiguousarray(gu, np.float32)
    rows = gu.shape[0]
    assert gu.shape[1] == 2 * ffn and (group == 0 or ffn % group == 0)
    out = np.empty((rows, ffn), np.uint16)
    lib().or_silu_mul_rows(_ptr(gu, ctypes.c_float), _ptr(out, ctypes.c_uint16), rows, ffn, group)
    return out


def silu_mul_bf16_elementwise(gu, ffn: int, group: int = 0):
    """The same stage element by element through or_silu (Python loop; small
    inputs only): the composition the row form must equal."""
    gu = np.ascontiguousarray(gu, np.float32)
    if group:
        blocks = gu.reshape(gu.shape[0], ffn // group, 2, group)
        g = np.ascontiguousarray(blocks[:, :, 0, :].reshape(gu.shape[0], ffn))
        u = np.ascontiguousarray(blocks[:, :, 1, :].reshape(gu.shape[0], ffn))
    else:
        g, u = gu[:, :ffn], gu[:, ffn:]
    f = lib().or_silu
    s = np.array([f(float(v)) for v in g.ravel()], np.float32).reshape(g.shape)
    return f32_to_bf16_bits_np((s * u).astype(np.float32))


def _rope_positions(lens, batch: int, tq: int):
    pos = np.empty(batch * tq, np.int64)
    for r in range(batch * tq):
        b, t = divmod(r, tq)
        pos[r] = int(lens[b]) - tq + t
    return pos


def _rotation_positions(lens, batch: int, tq: int, max_len):
    """The position each row is rotated at.  A row has a cache position only
    when its sequence holds at least tq positions (lens[b] >= tq) and the
    position lies before max_len (when given); a row without one (a sequence
    shorter than its query count, or a position past the cache) is rotated
    at position 0 and appends nothing -- this build's convention for rows
    the decoder never produces (the reference has no RoPE)."""
    pos = _rope_positions(lens, batch, tq)
    ok = np.array([int(lens[r // tq]) >= tq and (max_len is None or pos[r] < max_len)
                   for r in range(batch * tq)], bool)
    return pos, np.where(ok, pos, 0).astype(np.uint32)


def rope_qkv(qkv, inv_freq, lens, batch: int, tq: int, heads: int, head_dim: int, max_len=None):
    """-> (q bf16 [R][H*D], k bf16 [R][H][D], v bf16 [R][H][D], pos [R]);
    pos is the row's position lens[b] - tq + t, the rotation uses
    _rotation_positions."""
    qkv = np.ascontiguousarray(qkv, np.float32)
    R = batch * tq
    HD = heads * head_dim
    assert qkv.shape == (R, 3 * HD)
    pos, p32 = _rotation_positions(lens, batch, tq, max_len)
    inv = np.ascontiguousarray(inv_freq, np.float32)
    q = np.empty((R, HD), np.uint16)
    k = np.empty((R, heads, head_dim), np.uint16)
    v = np.empty((R, heads, head_dim), np.uint16)
    lib().or_rope_qkv_rows(_ptr(qkv, ctypes.c_float), _ptr(inv, ctypes.c_float),
                           _ptr(p32, ctypes.c_uint32), _ptr(q, ctypes.c_uint16),
                           _ptr(k, ctypes.c_uint16), _ptr(v, ctypes.c_uint16), R, heads, head_dim)
    return q, k, v, pos


def rope_qkv_per_head(qkv, inv_freq, lens, batch: int, tq: int, heads: int, head_dim: int,
                      max_len=None):
    """The same stage head by head through or_rope_f32 (small inputs only):
    the composition the row form must equal."""
    qkv = np.ascontiguousarray(qkv, np.float32)
    R = batch * tq
    HD = heads * head_dim
    q = np.empty((R, HD), np.uint16)
    k = np.empty((R, heads, head_dim), np.uint16)
    v = np.empty((R, heads, head_dim), np.uint16)
    pos, prot = _rotation_positions(lens, batch, tq, max_len)
    for r in range(R):
        p = int(prot[r])
        for h in range(heads):
            qs = qkv[r, h * head_dim:(h + 1) * head_dim]
            ks = qkv[r, HD + h * head_dim:HD + (h + 1) * head_dim]
            q[r, h * head_dim:(h + 1) * head_dim] = f32_to_bf16_bits_np(rope_f32(qs, p, inv_freq))
            k[r, h] = f32_to_bf16_bits_np(rope_f32(ks, p, inv_freq))
            v[r, h] = f32_to_bf16_bits_np(qkv[r, 2 * HD + h * head_dim:2 * HD + (h + 1) * head_dim])
    return q, k, v, pos


def attn_causal(q, kc, vc, lens, batch: int, tq: int, heads: int, head_dim: int, scale: float,
                threads=None):
    """q bf16 [B*Tq][H*D], caches [B][H][L][D] -> o f32 [B*Tq][H*D]."""
    q = np.asarray(q, np.uint16).reshape(batch, tq, heads, head_dim)
    lens = np.asarray(lens, np.int64)
    o = np.empty((batch, tq, heads, head_dim), np.float32)
    for t in range(tq):
        ln = np.maximum(lens - (tq - 1 - t), 0).astype(np.uint32)
        o[:, t] = attn_decode(np.ascontiguousarray(q[:, t]), kc, vc, ln, scale, threads=threads)
    return o.reshape(batch * tq, heads * head_dim)


def gemm(a16, b16, threads=None):
    """Sequential-order bf16 GEMM: (f32, bf16 bits)."""
    return matmul_bf16(a16, b16, threads=threads)


class DecoderOracle:
    """Whole-model sequential forward (all GEMMs in the reference's k order).
    Weights are host arrays of bf16 bits laid out as the library's
    (w_qkv [L][d][3d], w_o [L][d][d], w_gu [L][d][2F] with gate / up
    interleaved by 64 columns, w_down [L][F][d], embed [V][d], w_lm [d][V])."""

    def __init__(self, weights: dict, n_heads: int, head_dim: int, ffn: int, max_len: int,
                 rope_base: float = 10000.0, threads=None):
        self.w = weights
        self.threads = threads  # None: the oracle's default (all visible cores, <= 16)
        self.H, self.D, self.F, self.L = n_heads, head_dim, ffn, max_len
        self.d = n_heads * head_dim
        self.layers = len(weights["w_qkv"])
        from . import rope_inv_freq
        self.inv = rope_inv_freq(head_dim, rope_base)
        self.scale = float(np.float32(1.0 / np.sqrt(head_dim)))
        self.kc = None
        self.vc = None
        self.len = 0

    def _forward(self, tokens, batch: int, tq: int):
        H, D, d, F = self.H, self.D, self.d, self.F
        lens = np.full(batch, self.len + tq, np.int64)
        x = bf16_bits_to_f32(self.w["embed"][np.asarray(tokens, np.int64).ravel()])
        h = ffn_out = None
        for l in range(self.layers):
            if l == 0:
                _, xn = residual_rmsnorm_bf16(x)
            else:
                x, xn = residual_rmsnorm_bf16(h, ffn_out)
            qkv, _ = gemm(xn, self.w["w_qkv"][l], self.threads)
            q, k, v, pos = rope_qkv(qkv, self.inv, lens, batch, tq, H, D)
            for r in range(batch * tq):
                b = r // tq
                self.kc[l][b, :, pos[r]] = k[r]
                self.vc[l][b, :, pos[r]] = v[r]
            o = attn_causal(q, self.kc[l], self.vc[l], lens, batch, tq, H, D, self.scale,
                            self.threads)
            ap, _ = gemm(f32_to_bf16_bits_np(o), self.w["w_o"][l], self.threads)
            h, hn = residual_rmsnorm_bf16(x, ap)
            gu, _ = gemm(hn, self.w["w_gu"][l], self.threads)
            act = silu_mul_bf16(gu, F, 64)
            ffn_out, _ = gemm(act, self.w["w_down"][l], self.threads)
        last = np.arange(batch) * tq + (tq - 1)
        _, fxn = residual_rmsnorm_bf16(h[last], ffn_out[last])
        logits, _ = gemm(fxn, self.w["w_lm"], self.threads)
        nxt = np.array([argmax_f32(logits[b]) for b in range(batch)], np.uint32)
        self.len += tq
        return logits, nxt

    def prefill(self, tokens, batch: int, t: int):
        self.kc = [np.zeros((batch, self.H, self.L, self.D), np.uint16) for _ in range(self.layers)]
        self.vc = [np.zeros((batch, self.H, self.L, self.D), np.uint16) for _ in range(self.layers)]
        self.len = 0
        return self._forward(tokens, batch, t)

    def step(self, tokens, batch: int):
        return self._forward(tokens, batch, 1)

    def load_cache(self, kc, vc, length: int):
        """Start from caches filled elsewhere (e.g. by a GPU prefill):
        kc / vc per layer [batch][H][L][D] bf16, `length` positions valid."""
        self.kc = [np.array(k, np.uint16, copy=True) for k in kc]
        self.vc = [np.array(v, np.uint16, copy=True) for v in vc]
        self.len = length
