"""GPU parity of KV-cache decode attention: bitwise against the oracle.

The kernel reproduces every fold of the oracle in the same order (scores:
d ascending per position; max: exact parallel form of the sequential fold;
denominator and output: t ascending), so outputs must match bit for bit,
including ragged lengths, empty and single-position sequences, NaN scores,
and the full benchmark shape.
"""
import math

import numpy as np
import pytest

import catena_amd as ca
import oracle
from gpu_util import dev_normal_bf16, hash_bits, say

pytestmark = pytest.mark.gpu

D = 128


@pytest.fixture(scope="module", autouse=True)
def _init():
    say("init device 0")
    ca.init(0)


def _run(q, k, v, lens, B, H, L, scale):
    lb = ca.Buffer.from_array(np.asarray(lens, np.uint32))
    o = ca.Buffer(B * H * D * 4)
    ca.attn_decode_bf16(q, k, v, lb, o, B, H, L, D, scale)
    return o.read(np.float32, (B, H, D))


def _bitwise(got, want):
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn)
    assert np.array_equal(got[~gn].view(np.uint32), want[~wn].view(np.uint32))


@pytest.mark.parametrize("B,H,L,lens", [
    (2, 3, 100, [100, 37]),
    (4, 2, 257, [0, 1, 64, 257]),
    (3, 1, 1000, [65, 999, 128]),
    (1, 4, 4096, [4096]),
])
def test_attention_bitwise_small(B, H, L, lens):
    say(f"attention B={B} H={H} L={L} lens={lens}")
    seed = B * 1000 + H * 100 + L
    q = dev_normal_bf16(B * H * D, seed, 0)
    k = dev_normal_bf16(B * H * L * D, seed, 1)
    v = dev_normal_bf16(B * H * L * D, seed, 2)
    scale = 1.0 / math.sqrt(D)
    got = _run(q, k, v, lens, B, H, L, scale)
    want = oracle.attn_decode(q.read(np.uint16, (B, H, D)), k.read(np.uint16, (B, H, L, D)),
                              v.read(np.uint16, (B, H, L, D)), np.array(lens, np.uint32), scale)
    _bitwise(got, want)


def test_attention_nan_and_inf_scores():
    B, H, L = 1, 4, 70
    rng = np.random.default_rng(8)
    q16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B, H, D)).astype(np.float32))
    k32 = rng.normal(0, 1, (B, H, L, D)).astype(np.float32)
    k32[0, 0, 10, 5] = np.nan          # NaN in the middle: fold restarts after it
    k32[0, 1, L - 1, 0] = np.nan       # NaN at the last position: max is NaN
    k32[0, 2, 3, :] = 1e30             # +inf score
    k32[0, 3, :, :] = 0.0              # all scores equal (+0): ties
    k16 = oracle.f32_to_bf16_bits_np(k32)
    v16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B, H, L, D)).astype(np.float32))
    say("attention NaN / inf / tie scores")
    qb, kb, vb = ca.Buffer.from_array(q16), ca.Buffer.from_array(k16), ca.Buffer.from_array(v16)
    got = _run(qb, kb, vb, [L], B, H, L, 0.088388)
    want = oracle.attn_decode(q16, k16, v16, np.array([L], np.uint32), 0.088388)
    _bitwise(got, want)


def test_attention_full_shape_bitwise_and_run_to_run():
    B, H, L = 32, 32, 4096
    say("attention full shape B=32 H=32 L=4096")
    q = dev_normal_bf16(B * H * D, 41, 0)
    k = dev_normal_bf16(B * H * L * D, 41, 1)
    v = dev_normal_bf16(B * H * L * D, 41, 2)
    scale = float(np.float32(1.0 / math.sqrt(D)))
    lens = [L] * B
    got = _run(q, k, v, lens, B, H, L, scale)
    h = hash_bits(got)
    say("attention full shape run-to-run x3")
    for _ in range(3):
        assert hash_bits(_run(q, k, v, lens, B, H, L, scale)) == h
    say("attention full shape oracle compare")
    want = oracle.attn_decode(q.read(np.uint16, (B, H, D)), k.read(np.uint16, (B, H, L, D)),
                              v.read(np.uint16, (B, H, L, D)), np.array(lens, np.uint32), scale)
    _bitwise(got, want)


def test_attention_many_pairs_ragged():
    """1,028 (batch, head) pairs (more than four per CU): bitwise equal to
    the oracle with ragged lengths around the 32-row K blocks and 64-row V
    batches (0, 1, 31, 32, 33, 699 and 700 positions) and a NaN score."""
    B, H, L = 4, 257, 700
    lens = [0, 33, 699, 700]
    rng = np.random.default_rng(17)
    q16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B, H, D)).astype(np.float32))
    k32 = rng.normal(0, 1, (B, H, L, D)).astype(np.float32)
    k32[2, 5, 300, 7] = np.nan
    k16 = oracle.f32_to_bf16_bits_np(k32)
    v16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B, H, L, D)).astype(np.float32))
    say("attention many pairs B=4 H=257 L=700")
    qb, kb, vb = ca.Buffer.from_array(q16), ca.Buffer.from_array(k16), ca.Buffer.from_array(v16)
    scale = float(np.float32(1.0 / math.sqrt(D)))
    got = _run(qb, kb, vb, lens, B, H, L, scale)
    want = oracle.attn_decode(q16, k16, v16, np.array(lens, np.uint32), scale)
    _bitwise(got, want)
    say("attention many pairs, lengths 1 / 31 / 32")
    lens2 = [1, 31, 32, 700]
    got2 = _run(qb, kb, vb, lens2, B, H, L, scale)
    want2 = oracle.attn_decode(q16, k16, v16, np.array(lens2, np.uint32), scale)
    _bitwise(got2, want2)


def test_attention_program_abi():
    rt = ca.Runtime([])
    B, H, L = 2, 2, 50
    rng = np.random.default_rng(2)
    q16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B, H, D)).astype(np.float32))
    k16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B, H, L, D)).astype(np.float32))
    v16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B, H, L, D)).astype(np.float32))
    lens = np.array([50, 7], np.uint32)
    bufs = [ca.Buffer.from_array(x) for x in (q16, k16, v16, lens)]
    say("runtime exec attn.decode.via-mem")
    [res] = rt.exec("attn.decode.via-mem", [ca.Value.mem(b.mem) for b in bufs] +
                    [ca.Value.u64(x) for x in (B, H, L, D)] + [ca.Value.f32(0.125)], 1)
    got = ca.mem_to_array(res.get(), np.float32).reshape(B, H, D)
    _bitwise(got, oracle.attn_decode(q16, k16, v16, lens, 0.125))
    ca.mem_free(res.get())


@pytest.mark.parametrize("L,lens", [(640, [513, 640, 600, 577, 64, 65, 1, 0]),
                                    (2000, [2000, 1999, 1025, 256, 257, 255, 1024, 1500]),
                                    (600, [600, 384, 385, 383, 448, 63, 2, 599])])
def test_few_pairs_form_equals_many_pairs_form(L, lens):
    """Eight sequences x 16 heads (128 pairs) take the few-pair kernel's
    split form (two workgroups per pair); the same sequences inside a batch
    of 12 (192 pairs) its one-workgroup form, inside a batch of 40 (640
    pairs) the four-wave kernel: per (b, h) the outputs are the same bits,
    and all equal the oracle.  Lengths cross the 64-row blocks and the six score waves'
    rotation (384 rows), down to 1 and 0, around the 1024 switch of the
    denominator's chain, with ceil(L / 64) not a multiple of 4."""
    H = 16
    Bs, Bl = 8, 40
    seed = 77 + L
    q = dev_normal_bf16(Bl * H * D, seed, 0)
    k = dev_normal_bf16(Bl * H * L * D, seed, 1)
    v = dev_normal_bf16(Bl * H * L * D, seed, 2)
    scale = float(np.float32(1.0 / math.sqrt(D)))
    lens_l = list(lens) + [L] * (Bl - Bs)
    say(f"attention eight-wave form B={Bs} H={H} L={L}")
    small = _run(q, k, v, lens, Bs, H, L, scale)
    say(f"attention eight-wave form B=12 H={H} L={L}")
    mid = _run(q, k, v, lens_l[:12], 12, H, L, scale)
    say(f"attention four-wave form B={Bl} H={H} L={L}")
    large = _run(q, k, v, lens_l, Bl, H, L, scale)
    assert np.array_equal(small.view(np.uint32), mid[:Bs].view(np.uint32))
    assert np.array_equal(small.view(np.uint32), large[:Bs].view(np.uint32))
    want = oracle.attn_decode(q.read(np.uint16, (Bl, H, D))[:Bs], k.read(np.uint16, (Bl, H, L, D))[:Bs],
                              v.read(np.uint16, (Bl, H, L, D))[:Bs], np.array(lens, np.uint32), scale)
    _bitwise(small, want)


def test_attention_random_configs_bitwise():
    """Twelve seeded random configurations, B and H so that both the
    eight-wave few-pairs kernel (B * H <= 128, L >= 64) and the four-wave
    kernel run, random lengths in [0, L] (zeros and full lengths included)
    and random scales: every output bitwise the oracle's."""
    rng = np.random.default_rng(4242)
    for i in range(12):
        if i < 8:
            B, H = int(rng.integers(1, 9)), int(rng.integers(1, 17))
        else:
            B, H = int(rng.integers(9, 20)), int(rng.integers(9, 17))
        L = int(rng.integers(64, 1500))
        lens = rng.integers(0, L + 1, B)
        if i % 4 == 0:
            lens[0] = L
        if i % 4 == 1:
            lens[-1] = 0
        scale = float(np.float32(rng.uniform(0.05, 0.2)))
        say(f"attention random config B={B} H={H} L={L} lens={list(map(int, lens))} scale={scale}")
        seed = 5000 + i
        q = dev_normal_bf16(B * H * D, seed, 0)
        k = dev_normal_bf16(B * H * L * D, seed, 1)
        v = dev_normal_bf16(B * H * L * D, seed, 2)
        got = _run(q, k, v, lens, B, H, L, scale)
        want = oracle.attn_decode(q.read(np.uint16, (B, H, D)), k.read(np.uint16, (B, H, L, D)),
                                  v.read(np.uint16, (B, H, L, D)), np.asarray(lens, np.uint32), scale)
        _bitwise(got, want)


def test_few_pairs_form_ignores_rows_past_len():
    """K and V rows past each sequence's length hold NaN and infinities
    (inside the last, partial 64-row batch and beyond it); the eight-wave
    kernel folds the partial batch with those rows' products replaced by +0
    and gives the oracle's bits, which never read them."""
    B, H, L = 4, 8, 640
    lens = [600, 37, 64, 1]
    rng = np.random.default_rng(23)
    q16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B, H, D)).astype(np.float32))
    k32 = rng.normal(0, 1, (B, H, L, D)).astype(np.float32)
    v32 = rng.normal(0, 1, (B, H, L, D)).astype(np.float32)
    for b, n in enumerate(lens):
        k32[b, :, n:, ::2] = np.nan
        k32[b, :, n:, 1::2] = np.inf
        v32[b, :, n:, ::3] = np.nan
        v32[b, :, n:, 1::3] = -np.inf
    k16, v16 = oracle.f32_to_bf16_bits_np(k32), oracle.f32_to_bf16_bits_np(v32)
    qb, kb, vb = ca.Buffer.from_array(q16), ca.Buffer.from_array(k16), ca.Buffer.from_array(v16)
    say("attention eight-wave form, NaN / inf rows past len")
    got = _run(qb, kb, vb, lens, B, H, L, 0.088388)
    want = oracle.attn_decode(q16, k16, v16, np.array(lens, np.uint32), 0.088388)
    assert not np.isnan(want).any()
    _bitwise(got, want)


def test_few_pairs_form_nan_at_block_boundaries():
    """NaN and infinite scores at 64-row block boundaries (63 / 64, and 383 /
    384 where the six score waves' rotation wraps), several NaNs in one head
    with larger scores after the last, and a NaN at the last position,
    through the eight-wave kernel: bitwise the oracle."""
    B, H, L = 1, 6, 600
    rng = np.random.default_rng(18)
    q16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B, H, D)).astype(np.float32))
    k32 = rng.normal(0, 1, (B, H, L, D)).astype(np.float32)
    k32[0, 0, 63, 3] = np.nan
    k32[0, 1, 64, 0] = np.nan
    k32[0, 1, 300, :] = 1e30
    k32[0, 2, L - 1, 7] = np.nan
    k32[0, 3, 383, :] = 1e30
    k32[0, 3, 384, :] = 1e30   # two equal +inf scores: the first one wins the max
    k32[0, 4, 10, 1] = np.nan
    k32[0, 4, 200, 2] = np.nan
    k32[0, 4, 450, :] = 1e30   # after the last NaN: the max restarts there
    k32[0, 5, 0, 5] = np.nan
    k16 = oracle.f32_to_bf16_bits_np(k32)
    v16 = oracle.f32_to_bf16_bits_np(rng.normal(0, 1, (B, H, L, D)).astype(np.float32))
    qb, kb, vb = ca.Buffer.from_array(q16), ca.Buffer.from_array(k16), ca.Buffer.from_array(v16)
    say("attention eight-wave form NaN / inf at block boundaries")
    got = _run(qb, kb, vb, [L], B, H, L, 0.088388)
    want = oracle.attn_decode(q16, k16, v16, np.array([L], np.uint32), 0.088388)
    _bitwise(got, want)
