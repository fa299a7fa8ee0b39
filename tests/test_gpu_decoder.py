"""GPU parity of the decoder (catena_mi355x_decoder_*).

Stage by stage: every elementwise / fold stage of a forward must equal the
oracle applied to the GPU's own previous stage bit for bit (embedding,
RMSNorm with residual, RoPE + cache append, attention, SwiGLU, argmax), and
every GEMM stage must sit inside the MFMA-order bound of the bf16 contraction
(|C - AB| <= 8 (K/32 + 1) u sum|A||B|).  This pins the wiring as well as
the kernels: a stage fed from the wrong buffer, position or layer fails.

End to end: a two-layer model against the oracle's whole sequential forward
(all GEMMs in the reference's k order), logits within a stated tolerance and
greedy tokens equal wherever the oracle's top-2 margin exceeds it; and two
runs must agree bit for bit.
"""
import numpy as np
import pytest

import catena_amd as ca
import oracle
from oracle import decoder as od
from gpu_util import as_f32, gemm_within_bound, say

pytestmark = pytest.mark.gpu

D = 128


@pytest.fixture(scope="module", autouse=True)
def _init():
    say("init device 0")
    ca.init(0)


def _bitwise(got, want):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    if got.dtype == np.float32:
        gn, wn = np.isnan(got), np.isnan(want)
        assert np.array_equal(gn, wn)
        got, want = got[~gn].view(np.uint32), want[~wn].view(np.uint32)
    assert np.array_equal(got, want), int(np.sum(got != want))


class Tiny:
    H, F, V, B, T, L, layers = 2, 512, 512, 2, 16, 24, 1
    d = H * D


def _weights(dec, cfg):
    d, F, V = cfg.d, cfg.F, cfg.V
    w = {"embed": dec.read(ca.DEC_EMBED, np.uint16).reshape(V, d),
         "w_lm": dec.read(ca.DEC_W_LM, np.uint16).reshape(d, V)}
    for name, which, shape in [("w_qkv", ca.DEC_W_QKV, (d, 3 * d)), ("w_o", ca.DEC_W_O, (d, d)),
                               ("w_gu", ca.DEC_W_GU, (d, 2 * F)), ("w_down", ca.DEC_W_DOWN, (F, d))]:
        w[name] = [dec.read(which, np.uint16, layer=l).reshape(shape) for l in range(cfg.layers)]
    return w


def _check_forward(dec, cfg, w, tokens, tq, cache_len):
    """Check the last forward (rows = B * tq, cache holding cache_len positions
    after it) stage by stage, through the last layer (whose input x is the
    embedding with one layer, else the previous layer's residual stream,
    checked through its RMSNorm); returns the GPU's next tokens."""
    d, F, B, H = cfg.d, cfg.F, cfg.B, cfg.H
    R = B * tq
    lay = cfg.layers - 1
    lens = np.full(B, cache_len, np.int64)
    rd = lambda which, dt, shape: dec.read(which, dt, layer=lay).reshape(shape)  # noqa: E731
    toks = np.asarray(tokens, np.int64).ravel()
    if lay == 0 and tq == 1:
        # a decode step gathers layer 0's normalized rows from the table of
        # normalized embedding rows (row V: the out-of-range row) and reads x
        # as the embedding rows: it writes neither X nor XN
        X = as_f32(w["embed"][toks])
        tab = dec.read(ca.DEC_EMBED_NORM, np.uint16).reshape(cfg.V + 1, d)
        XN = tab[np.minimum(toks, cfg.V)]
    else:
        X = rd(ca.DEC_X, np.float32, (R, d))
        if lay == 0:
            _bitwise(X, as_f32(w["embed"][toks]))
        XN = rd(ca.DEC_XN, np.uint16, (R, d))
    _bitwise(XN, od.residual_rmsnorm_bf16(X)[1])
    if tq > 1 and R % 256 == 0 and d % 128 == 0:
        # prefill with RoPE and the cache append in W_qkv's GEMM epilogue:
        # the f32 product is never written; the plain GEMM recomputes it
        # (the same tile kernel's order, so the same bits) to check q and
        # the caches against
        qkv = ca.Buffer(R * 3 * d * 4)
        ca.gemm_bf16(ca.Buffer.from_array(XN), ca.Buffer.from_array(w["w_qkv"][lay]), qkv, R, 3 * d,
                     d, out_f32=True)
        QKV = qkv.read(np.float32, (R, 3 * d))
    else:
        QKV = rd(ca.DEC_QKV, np.float32, (R, 3 * d))
    gemm_within_bound(XN, w["w_qkv"][lay], QKV)
    inv = dec.read(ca.DEC_INV_FREQ, np.float32)
    q, k, v, pos = od.rope_qkv(QKV, inv, lens, B, tq, H, D)
    Q = rd(ca.DEC_Q, np.uint16, (R, d))
    _bitwise(Q, q)
    kc = rd(ca.DEC_K_CACHE, np.uint16, (B, H, cfg.L, D))
    vc = rd(ca.DEC_V_CACHE, np.uint16, (B, H, cfg.L, D))
    for r in range(R):
        _bitwise(kc[r // tq, :, pos[r]], k[r])
        _bitwise(vc[r // tq, :, pos[r]], v[r])
    ATT = rd(ca.DEC_ATTN, np.uint16, (R, d))
    o = od.attn_causal(Q, kc, vc, lens, B, tq, H, D, float(np.float32(1 / np.sqrt(D))))
    _bitwise(ATT, oracle.f32_to_bf16_bits_np(o))
    AP = rd(ca.DEC_ATTN_PROJ, np.float32, (R, d))
    gemm_within_bound(ATT, w["w_o"][lay], AP)
    Hh = rd(ca.DEC_H, np.float32, (R, d))
    h, hn = od.residual_rmsnorm_bf16(X, AP)
    _bitwise(Hh, h)
    HN = rd(ca.DEC_HN, np.uint16, (R, d))
    _bitwise(HN, hn)
    if tq > 1 and R % 256 == 0 and d % 128 == 0 and (2 * F) % 128 == 0:
        # prefill with the SwiGLU gate in W_gu's GEMM epilogue: the f32
        # product is never written; the plain GEMM recomputes it (the same
        # tile kernel's order, so the same bits) to check act against
        gu = ca.Buffer(R * 2 * F * 4)
        ca.gemm_bf16(ca.Buffer.from_array(HN), ca.Buffer.from_array(w["w_gu"][lay]), gu, R, 2 * F, d,
                     out_f32=True)
        GU = gu.read(np.float32, (R, 2 * F))
    else:
        GU = rd(ca.DEC_GU, np.float32, (R, 2 * F))
    gemm_within_bound(HN, w["w_gu"][lay], GU)
    ACT = rd(ca.DEC_ACT, np.uint16, (R, F))
    _bitwise(ACT, od.silu_mul_bf16(GU, F, 64))
    FO = rd(ca.DEC_FFN_OUT, np.float32, (R, d))
    last = np.arange(B) * tq + (tq - 1)
    if tq > 1 and R % 256 == 0 and d % 256 == 0 and F % 256 == 0 and (R // 256) * (d // 256) <= 128:
        # prefill with W_down as two k-half partials, added by the final norm,
        # which writes the sums of the rows it reads (each sequence's last)
        gemm_within_bound(ACT[last], w["w_down"][lay], FO[last])
    else:
        gemm_within_bound(ACT, w["w_down"][lay], FO)
    fh, fxn = od.residual_rmsnorm_bf16(Hh[last], FO[last])
    _bitwise(rd(ca.DEC_FINAL_H, np.float32, (B, d)), fh)
    FXN = rd(ca.DEC_FINAL_XN, np.uint16, (B, d))
    _bitwise(FXN, fxn)
    LG = rd(ca.DEC_LOGITS, np.float32, (B, cfg.V))
    gemm_within_bound(FXN, w["w_lm"], LG)
    assert list(dec.read(ca.DEC_LENS, np.uint32)) == [cache_len] * B
    return np.array([oracle.argmax_f32(LG[b]) for b in range(B)], np.uint32)


def _check_step_qkv_token(dec, cfg, tab, w_qkv_f64, tokens_in, cache_len, token_out):
    """The per-step check of a decode step that needs no attention oracle:
    the step's W_qkv product (of the rows of `tab`, the normalized embedding
    table, that the step's input tokens select) within the GEMM bound; q and the new K / V cache
    rows at pos = cache_len - 1 bitwise the oracle's RoPE of that product;
    the greedy token the oracle's argmax of the GPU logits."""
    d, B, H = cfg.d, cfg.B, cfg.H
    toks = np.asarray(tokens_in, np.int64).ravel()
    XN = tab[np.minimum(toks, cfg.V)]
    QKV = dec.read(ca.DEC_QKV, np.float32).reshape(B, 3 * d)
    af = as_f32(XN).astype(np.float64)
    bound = 8 * (d / 32 + 1) * 2.0 ** -24 * (np.abs(af) @ np.abs(w_qkv_f64))
    assert np.all(np.abs(QKV.astype(np.float64) - af @ w_qkv_f64) <= bound)
    lens = np.full(B, cache_len, np.int64)
    inv = dec.read(ca.DEC_INV_FREQ, np.float32)
    q, k, v, pos = od.rope_qkv(QKV, inv, lens, B, 1, H, D)
    assert np.all(pos == cache_len - 1)
    _bitwise(dec.read(ca.DEC_Q, np.uint16).reshape(B, d), q)
    kc = dec.read(ca.DEC_K_CACHE, np.uint16).reshape(B, H, cfg.L, D)
    vc = dec.read(ca.DEC_V_CACHE, np.uint16).reshape(B, H, cfg.L, D)
    _bitwise(kc[:, :, cache_len - 1], k.reshape(B, H, D))
    _bitwise(vc[:, :, cache_len - 1], v.reshape(B, H, D))
    LG = dec.read(ca.DEC_LOGITS, np.float32).reshape(B, cfg.V)
    want = np.array([oracle.argmax_f32(LG[b]) for b in range(B)], np.uint32)
    assert np.array_equal(np.asarray(token_out, np.uint32), want)


def test_decoder_stagewise_prefill_and_steps():
    cfg = Tiny
    dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
    dec.init_weights(seed=5, std=0.02)
    w = _weights(dec, cfg)
    tokens = np.random.default_rng(1).integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
    tb = ca.Buffer.from_array(tokens)
    nxt = ca.Buffer(cfg.B * 4)
    say("decoder prefill (tiny)")
    dec.prefill(tb, cfg.B, cfg.T, nxt)
    want_next = _check_forward(dec, cfg, w, tokens, cfg.T, cfg.T)
    got_next = nxt.read(np.uint32)
    assert np.array_equal(got_next, want_next)
    prev = got_next
    for s in range(3):
        out = ca.Buffer(cfg.B * 4)
        say(f"decoder step {s}")
        dec.generate(1, out)
        want = _check_forward(dec, cfg, w, prev, 1, cfg.T + s + 1)
        got = out.read(np.uint32)
        assert np.array_equal(got, want)
        prev = got
    # the cache is full after L - T more steps; one more must be refused
    steps_left = cfg.L - (cfg.T + 3)
    buf = ca.Buffer(cfg.B * 4 * (steps_left + 1))
    with pytest.raises(ca.CatenaError):
        dec.generate(steps_left + 1, buf)
    dec.close()


def test_decoder_embed_norm_table_and_rebuild():
    """The table of normalized embedding rows that a decode step gathers
    layer 0's input from: every row bitwise the oracle's rmsnorm of the
    widened embedding row, row V all NaN; after the embedding is rewritten
    through decoder_tensor, the next forward rebuilds it, and the decode
    step then checks stage by stage against the new weights."""
    cfg = Tiny
    dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
    dec.init_weights(seed=9, std=0.02)
    say("normalized embedding table after init_weights")
    tab = dec.read(ca.DEC_EMBED_NORM, np.uint16).reshape(cfg.V + 1, cfg.d)
    emb = dec.read(ca.DEC_EMBED, np.uint16).reshape(cfg.V, cfg.d)
    _bitwise(tab[:cfg.V], od.residual_rmsnorm_bf16(as_f32(emb))[1])
    assert np.isnan(as_f32(tab[cfg.V])).all()
    # a new embedding (rows of very different scales) written through the
    # tensor handle
    rng = np.random.default_rng(19)
    new = oracle.f32_to_bf16_bits_np(
        (rng.normal(0, 1, (cfg.V, cfg.d)) * np.exp(rng.normal(0, 3, (cfg.V, 1)))).astype(np.float32))
    ca.mem_write(dec.tensor(ca.DEC_EMBED), new)
    w = _weights(dec, cfg)
    assert np.array_equal(w["embed"], new)
    tokens = rng.integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
    nxt = ca.Buffer(cfg.B * 4)
    say("prefill and one step after rewriting the embedding")
    dec.prefill(ca.Buffer.from_array(tokens), cfg.B, cfg.T, nxt)
    tab = dec.read(ca.DEC_EMBED_NORM, np.uint16).reshape(cfg.V + 1, cfg.d)
    _bitwise(tab[:cfg.V], od.residual_rmsnorm_bf16(as_f32(new))[1])
    prev = nxt.read(np.uint32)
    out = ca.Buffer(cfg.B * 4)
    dec.generate(1, out)
    want = _check_forward(dec, cfg, w, prev, 1, cfg.T + 1)
    assert np.array_equal(out.read(np.uint32), want)
    dec.close()


def test_decoder_embedding_written_through_retained_handle():
    """A handle to the embedding taken before any forward and written after
    one (no further decoder_tensor call): the next generate call rebuilds the
    normalized table, so the decode step's gathered layer-0 input and its
    residual both follow the new embedding (checked stage by stage)."""
    cfg = Tiny
    dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
    dec.init_weights(seed=23, std=0.02)
    handle = dec.tensor(ca.DEC_EMBED)
    rng = np.random.default_rng(23)
    tokens = rng.integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
    nxt = ca.Buffer(cfg.B * 4)
    say("prefill, then write the embedding through a handle kept from before it")
    dec.prefill(ca.Buffer.from_array(tokens), cfg.B, cfg.T, nxt)
    prev = nxt.read(np.uint32)
    for s_ in range(2):
        new = oracle.f32_to_bf16_bits_np(
            (rng.normal(0, 1, (cfg.V, cfg.d)) * np.exp(rng.normal(0, 2, (cfg.V, 1)))).astype(np.float32))
        ca.mem_write(handle, new)
        out = ca.Buffer(cfg.B * 4)
        say(f"decode step {s_} after the write")
        dec.generate(1, out)
        w = _weights(dec, cfg)
        assert np.array_equal(w["embed"], new)
        want = _check_forward(dec, cfg, w, prev, 1, cfg.T + s_ + 1)
        got = out.read(np.uint32)
        assert np.array_equal(got, want)
        prev = got
    dec.close()


class FewPartial(Tiny):
    """max_len >= 64, so a decode step runs the eight-wave attention on
    W_qkv's partials; T = 37 puts the new positions inside a partial 64-row
    V batch and at many rows of the score blocks."""
    H, F, V, B, T, L, layers = 2, 512, 512, 2, 37, 100, 1
    d = H * D


def test_decoder_few_pair_attention_partial_batches_stagewise():
    """Decode steps at positions 37 .. 66 (the new key and value put into the
    registers / the LDS batch at every row of a partial block, and across the
    64-position boundary), each checked stage by stage."""
    cfg = FewPartial
    dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
    dec.init_weights(seed=29, std=0.02)
    w = _weights(dec, cfg)
    tokens = np.random.default_rng(29).integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
    nxt = ca.Buffer(cfg.B * 4)
    say("prefill (max_len 100, T 37)")
    dec.prefill(ca.Buffer.from_array(tokens), cfg.B, cfg.T, nxt)
    prev = nxt.read(np.uint32)
    for s_ in range(30):
        out = ca.Buffer(cfg.B * 4)
        say(f"decode step at position {cfg.T + s_} (max_len 100)")
        dec.generate(1, out)
        want = _check_forward(dec, cfg, w, prev, 1, cfg.T + s_ + 1)
        got = out.read(np.uint32)
        assert np.array_equal(got, want)
        prev = got
    dec.close()


@pytest.mark.parametrize("cfg", [Tiny, FewPartial], ids=["tiny", "few_pair"])
def test_decoder_generate_n_equals_n_single_steps(cfg):
    """generate(N) composes each step's token from the LM head's column-block
    summaries inside the next step's W_qkv (the deferred argmax); generate(1)
    composes it in its own launch.  Two decoders from the same seeds: the
    tokens of one generate(6) and the logits after it equal those of six
    generate(1) calls bit for bit."""
    tokens = np.random.default_rng(31).integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
    runs = []
    for mode in ("one call", "single steps"):
        dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
        dec.init_weights(seed=31, std=0.02)
        nxt = ca.Buffer(cfg.B * 4)
        dec.prefill(ca.Buffer.from_array(tokens), cfg.B, cfg.T, nxt)
        say(f"generate 6 steps ({mode})")
        if mode == "one call":
            out = ca.Buffer(6 * cfg.B * 4)
            dec.generate(6, out)
            toks = out.read(np.uint32, (6, cfg.B))
        else:
            toks = []
            for _ in range(6):
                out = ca.Buffer(cfg.B * 4)
                dec.generate(1, out)
                toks.append(out.read(np.uint32))
            toks = np.stack(toks)
        runs.append((toks, dec.read(ca.DEC_LOGITS, np.float32)))
        dec.close()
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1].view(np.uint32), runs[1][1].view(np.uint32))


def test_decoder_random_configs_stagewise():
    """Eight seeded random small models (1-3 heads, SwiGLU width, vocabulary,
    batch, prompt length 1-60 with partial 16-query blocks among them, one
    or two layers, cache 4-80 positions past the prompt): the prefill and
    three decode steps, each checked stage by stage against the oracle, and
    the greedy tokens against the oracle's argmax of the GPU logits."""
    rng = np.random.default_rng(555)
    prompts = [14, 43, 1, 27]  # partial blocks of 14 and 11 queries, one row, 27 = 16 + 11
    for i in range(8):
        H = int(rng.integers(1, 4))
        cfg = type(f"Rand{i}", (), dict(
            H=H, d=H * D, F=64 * int(rng.integers(1, 12)), V=8 * int(rng.integers(8, 200)),
            B=int(rng.integers(1, 5)), layers=int(rng.integers(1, 3)),
            T=prompts[i] if i < len(prompts) else int(rng.integers(1, 61))))
        cfg.L = cfg.T + int(rng.integers(4, 81))
        say(f"random decoder {i}: d={cfg.d} F={cfg.F} V={cfg.V} B={cfg.B} layers={cfg.layers} "
            f"T={cfg.T} L={cfg.L}")
        dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
        dec.init_weights(seed=600 + i, std=0.02)
        w = _weights(dec, cfg)
        tokens = rng.integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
        nxt = ca.Buffer(cfg.B * 4)
        dec.prefill(ca.Buffer.from_array(tokens), cfg.B, cfg.T, nxt)
        want = _check_forward(dec, cfg, w, tokens, cfg.T, cfg.T)
        prev = nxt.read(np.uint32)
        assert np.array_equal(prev, want)
        for s_ in range(3):
            out = ca.Buffer(cfg.B * 4)
            dec.generate(1, out)
            want = _check_forward(dec, cfg, w, prev, 1, cfg.T + s_ + 1)
            got = out.read(np.uint32)
            assert np.array_equal(got, want), (i, s_)
            prev = got
        dec.close()


def test_decoder_random_large_batches_stagewise():
    """Random models with batches past the decode GEMM's 16 rows (17-40
    sequences: the projections and the LM head take the tile / edge GEMMs and
    the argmax its own launch) and up to three layers: prefill and two
    decode steps, stage by stage."""
    rng = np.random.default_rng(556)
    for i in range(3):
        H = int(rng.integers(1, 3))
        cfg = type(f"RandBig{i}", (), dict(
            H=H, d=H * D, F=64 * int(rng.integers(1, 8)), V=8 * int(rng.integers(8, 100)),
            B=int(rng.integers(17, 41)), layers=int(rng.integers(1, 4)), T=int(rng.integers(1, 20))))
        cfg.L = cfg.T + int(rng.integers(3, 40))
        say(f"random decoder, large batch {i}: d={cfg.d} F={cfg.F} V={cfg.V} B={cfg.B} "
            f"layers={cfg.layers} T={cfg.T} L={cfg.L}")
        dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
        dec.init_weights(seed=700 + i, std=0.02)
        w = _weights(dec, cfg)
        tokens = rng.integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
        nxt = ca.Buffer(cfg.B * 4)
        dec.prefill(ca.Buffer.from_array(tokens), cfg.B, cfg.T, nxt)
        prev = nxt.read(np.uint32)
        assert np.array_equal(prev, _check_forward(dec, cfg, w, tokens, cfg.T, cfg.T))
        for s_ in range(2):
            out = ca.Buffer(cfg.B * 4)
            dec.generate(1, out)
            want = _check_forward(dec, cfg, w, prev, 1, cfg.T + s_ + 1)
            got = out.read(np.uint32)
            assert np.array_equal(got, want), (i, s_)
            prev = got
        dec.close()


def test_decoder_random_long_caches_stagewise():
    """Random models whose caches pass the prefill kernel's LDS limit (max_len
    900-1300: the causal attention takes the one-query kernel) with prompts
    of 100-400 positions: prefill and two decode steps, stage by stage."""
    rng = np.random.default_rng(557)
    for i in range(2):
        H = int(rng.integers(1, 3))
        cfg = type(f"RandLong{i}", (), dict(
            H=H, d=H * D, F=64 * int(rng.integers(1, 6)), V=8 * int(rng.integers(8, 64)),
            B=int(rng.integers(1, 4)), layers=1, T=int(rng.integers(100, 401))))
        cfg.L = int(rng.integers(900, 1301))
        say(f"random decoder, long cache {i}: d={cfg.d} F={cfg.F} V={cfg.V} B={cfg.B} T={cfg.T} L={cfg.L}")
        dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
        dec.init_weights(seed=710 + i, std=0.02)
        w = _weights(dec, cfg)
        tokens = rng.integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
        nxt = ca.Buffer(cfg.B * 4)
        dec.prefill(ca.Buffer.from_array(tokens), cfg.B, cfg.T, nxt)
        prev = nxt.read(np.uint32)
        assert np.array_equal(prev, _check_forward(dec, cfg, w, tokens, cfg.T, cfg.T))
        for s_ in range(2):
            out = ca.Buffer(cfg.B * 4)
            dec.generate(1, out)
            want = _check_forward(dec, cfg, w, prev, 1, cfg.T + s_ + 1)
            got = out.read(np.uint32)
            assert np.array_equal(got, want), (i, s_)
            prev = got
        dec.close()


class C5Step(Tiny):
    H, F, V, B, T, L, layers = 16, 5632, 32000, 8, 4, 8, 1
    d = H * D


def test_decoder_c5_width_decode_step_stagewise():
    """A decode step at the C5 model width (d 2048, SwiGLU 5632, vocab 32000,
    batch 8: the shapes the decode-GEMM epilogues and split-K run at in the
    benchmark), stage by stage, as above."""
    cfg = C5Step
    dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
    dec.init_weights(seed=11, std=0.02)
    w = _weights(dec, cfg)
    tokens = np.random.default_rng(3).integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
    nxt = ca.Buffer(cfg.B * 4)
    say("decoder prefill (C5 width)")
    dec.prefill(ca.Buffer.from_array(tokens), cfg.B, cfg.T, nxt)
    prev = nxt.read(np.uint32)
    out = ca.Buffer(cfg.B * 4)
    say("decoder step (C5 width)")
    dec.generate(1, out)
    want = _check_forward(dec, cfg, w, prev, 1, cfg.T + 1)
    assert np.array_equal(out.read(np.uint32), want)
    dec.close()


class Wide2L(Tiny):
    H, F, V, T, L, layers = 16, 512, 512, 2, 6, 2
    d = H * D


@pytest.mark.parametrize("batch", [3, 16])
def test_decoder_two_layers_decode_steps_stagewise(batch):
    """Decode steps at d 2048 with two layers (the second layer's input is the
    first one's residual stream, checked through its RMSNorm), stage by stage
    as above, for a ragged batch and the largest batch the decode-GEMM
    epilogues take (16 rows)."""
    cfg = type("Wide2LBatch", (Wide2L,), {"B": batch})
    dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
    dec.init_weights(seed=13, std=0.02)
    w = _weights(dec, cfg)
    tokens = np.random.default_rng(4).integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
    nxt = ca.Buffer(cfg.B * 4)
    say(f"decoder prefill (d 2048, two layers, batch {batch})")
    dec.prefill(ca.Buffer.from_array(tokens), cfg.B, cfg.T, nxt)
    prev = nxt.read(np.uint32)
    for s_ in range(2):
        out = ca.Buffer(cfg.B * 4)
        say(f"decoder step {s_} (d 2048, two layers, batch {batch})")
        dec.generate(1, out)
        want = _check_forward(dec, cfg, w, prev, 1, cfg.T + s_ + 1)
        got = out.read(np.uint32)
        assert np.array_equal(got, want)
        prev = got
    dec.close()


class Prefill256(Tiny):
    H, F, V, B, T, L, layers = 2, 512, 512, 16, 16, 20, 1
    d = H * D


def test_decoder_prefill_fused_swiglu_stagewise():
    """A prefill of 256 rows, where W_gu's GEMM carries the SwiGLU gate in
    its epilogue (act only, no f32 product), then a decode step: stage by
    stage as above."""
    cfg = Prefill256
    dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
    dec.init_weights(seed=17, std=0.02)
    w = _weights(dec, cfg)
    tokens = np.random.default_rng(6).integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
    nxt = ca.Buffer(cfg.B * 4)
    say("decoder prefill of 256 rows (fused SwiGLU)")
    dec.prefill(ca.Buffer.from_array(tokens), cfg.B, cfg.T, nxt)
    want = _check_forward(dec, cfg, w, tokens, cfg.T, cfg.T)
    got = nxt.read(np.uint32)
    assert np.array_equal(got, want)
    out = ca.Buffer(cfg.B * 4)
    say("decoder step after the 256-row prefill")
    dec.generate(1, out)
    want = _check_forward(dec, cfg, w, got, 1, cfg.T + 1)
    assert np.array_equal(out.read(np.uint32), want)
    dec.close()


def test_decoder_create_rejects_unsupported_configs():
    """A cache longer than the attention's LDS holds, or a batch beyond the
    lens table's bound, fails at create with CATENA_ERR_UNSUPPORTED."""
    with pytest.raises(ca.CatenaError):
        ca.Decoder(256, 2, 512, 1, 512, 2, 40000)
    with pytest.raises(ca.CatenaError):
        ca.Decoder(256, 2, 512, 1, 512, 5000, 16)


def _run_model(cfg, tokens, steps, seed):
    dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
    dec.init_weights(seed=seed, std=0.02)
    tb = ca.Buffer.from_array(tokens)
    nxt = ca.Buffer(cfg.B * 4)
    dec.prefill(tb, cfg.B, cfg.T, nxt)
    logits = [dec.read(ca.DEC_LOGITS, np.float32).reshape(cfg.B, cfg.V)]
    toks = [nxt.read(np.uint32)]
    for _ in range(steps):
        out = ca.Buffer(cfg.B * 4)
        dec.generate(1, out)
        logits.append(dec.read(ca.DEC_LOGITS, np.float32).reshape(cfg.B, cfg.V))
        toks.append(out.read(np.uint32))
    return dec, logits, toks


class TwoLayer(Tiny):
    layers, T, L = 2, 12, 20


def test_decoder_two_layers_against_sequential_oracle_and_run_to_run():
    cfg = TwoLayer
    tokens = np.random.default_rng(2).integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
    say("decoder two-layer run A")
    dec, logits, toks = _run_model(cfg, tokens, 4, seed=9)
    w = _weights(dec, cfg)
    dec.close()
    say("decoder two-layer run B (run-to-run)")
    dec2, logits2, toks2 = _run_model(cfg, tokens, 4, seed=9)
    dec2.close()
    for a, b in zip(logits, logits2):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for a, b in zip(toks, toks2):
        assert np.array_equal(a, b)

    say("decoder two-layer oracle forward")
    ora = od.DecoderOracle(w, cfg.H, D, cfg.F, cfg.L)
    ol, on = ora.prefill(tokens, cfg.B, cfg.T)
    # Tolerance: GEMM order differences change some bf16 roundings of the
    # activations (one bf16 ulp = 2^-8 relative); 3% of the logit scale.
    for step in range(5):
        scale = float(np.abs(ol).max())
        tol = 0.03 * scale
        assert np.abs(logits[step] - ol).max() <= tol, (step, float(np.abs(logits[step] - ol).max()), scale)
        srt = np.sort(ol, axis=1)
        margin = srt[:, -1] - srt[:, -2]
        clear = margin > 2 * tol
        assert np.array_equal(toks[step][clear], on[clear])
        if not np.all(clear) or step == 4:
            break
        ol, on = ora.step(toks[step], cfg.B)


class C5:
    """d 2048, 16 heads of 128, SwiGLU 5632, vocab 32000,
    one block, batch 8, a 512-token prefill then 128 greedy steps (the cache
    holds 640 positions after the last one)."""
    H, F, V, B, T, layers = 16, 5632, 32000, 8, 512, 1
    d = H * D
    steps = 128
    L = T + steps


def test_decoder_c5_full_workload_stagewise():
    """The C5 workload as bench.py runs it (same seeds): the 4096-row prefill
    (the 256-row-tile GEMMs, the SwiGLU-fused W_gu GEMM, the 16-query-block
    prefill attention over 512 positions) checked stage by stage; then the
    128 greedy steps one generate(1) call at a time, each one's W_qkv
    product, q, appended K / V cache rows (positions 512 .. 639) and token
    checked against the oracle, and the first and last steps checked stage
    by stage.  A second decoder from the same seeds runs the steps as one
    generate(127) call (the deferred argmax inside W_qkv) and one
    generate(1): its tokens and final logits equal the first one's bit for
    bit."""
    cfg = C5
    say("C5 decoder: create + init weights")
    dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
    dec.init_weights(seed=51, std=0.02)
    w = _weights(dec, cfg)
    w_qkv64 = as_f32(w["w_qkv"][0]).astype(np.float64)
    tab = dec.read(ca.DEC_EMBED_NORM, np.uint16).reshape(cfg.V + 1, cfg.d)
    _bitwise(tab[:cfg.V], od.residual_rmsnorm_bf16(as_f32(w["embed"]))[1])
    tokens = np.random.default_rng(51).integers(0, cfg.V, (cfg.B, cfg.T)).astype(np.uint32)
    tb = ca.Buffer.from_array(tokens)
    nxt = ca.Buffer(cfg.B * 4)
    say("C5 decoder: prefill 8 x 512")
    dec.prefill(tb, cfg.B, cfg.T, nxt)
    say("C5 decoder: prefill stagewise check")
    want = _check_forward(dec, cfg, w, tokens, cfg.T, cfg.T)
    prev = nxt.read(np.uint32)
    assert np.array_equal(prev, want)
    toks = []
    for s_ in range(cfg.steps):
        out = ca.Buffer(cfg.B * 4)
        if s_ % 16 == 0:
            say(f"C5 decoder: step {s_ + 1} of {cfg.steps} (cache length {cfg.T + s_ + 1})")
        dec.generate(1, out)
        got = out.read(np.uint32)
        if s_ in (0, cfg.steps - 1):
            want = _check_forward(dec, cfg, w, prev, 1, cfg.T + s_ + 1)
            assert np.array_equal(got, want)
        else:
            _check_step_qkv_token(dec, cfg, tab, w_qkv64, prev, cfg.T + s_ + 1, got)
        toks.append(got)
        prev = got
    toks = np.stack(toks)
    assert toks.max() < cfg.V
    final_logits = dec.read(ca.DEC_LOGITS, np.float32)
    dec.close()

    say("C5 decoder B: prefill, generate(127) + generate(1)")
    dec = ca.Decoder(cfg.d, cfg.H, cfg.F, cfg.layers, cfg.V, cfg.B, cfg.L)
    dec.init_weights(seed=51, std=0.02)
    dec.prefill(tb, cfg.B, cfg.T, nxt)
    out = ca.Buffer((cfg.steps - 1) * cfg.B * 4)
    dec.generate(cfg.steps - 1, out)
    last = ca.Buffer(cfg.B * 4)
    dec.generate(1, last)
    toks_b = np.concatenate([out.read(np.uint32, (cfg.steps - 1, cfg.B)),
                             last.read(np.uint32, (1, cfg.B))])
    assert np.array_equal(toks_b, toks)
    assert np.array_equal(dec.read(ca.DEC_LOGITS, np.float32).view(np.uint32),
                          final_logits.view(np.uint32))
    dec.close()
