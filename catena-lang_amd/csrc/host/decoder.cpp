// Llama-style decoder built from the library's kernels: the model the two
// hot contractions (bf16 GEMM, KV-cache attention) serve.  No reference
// counterpart; its pieces mirror the reference's stdlib ops (nn.rmsnorm,
// nn.silu, math.sin-approx-full, tensor.argmax-f32) bit for bit, and the
// GEMMs follow the bf16 contraction contract of catena_mi355x_gemm_bf16.
//
// Everything after create() is stream-ordered on the library stream with no
// host synchronisation: prefill and the greedy generate loop enqueue their
// kernels and return; the argmax of step s feeds the embedding gather of
// step s + 1 on the device.  Sequence lengths are uniform across the batch,
// so the per-sequence lengths a step needs are rows of a table uploaded once
// (lens_table[t][b] = t).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "internal.h"

using namespace catena;

struct catena_decoder {
  catena_decoder_config_t cfg{};
  uint64_t d = 0, f = 0;
  // weights and caches
  void* embed = nullptr;
  // bf16 rmsnorm of every embedding row ([vocab + 1][d], the last row NaN),
  // rebuilt before a forward when the embedding may have changed
  void* embed_norm = nullptr;
  bool embed_norm_stale = true;
  // set once decoder_tensor has handed out the embedding: the caller may
  // write through that handle at any time, so from then on every prefill
  // and generate call rebuilds the table first
  bool embed_exposed = false;
  void* w_lm = nullptr;
  void* inv_freq = nullptr;
  void* rope_tab = nullptr;  // [max_len][head_dim / 2][2] f32: (cos, sin) per position and pair
  // a decode step's W_qkv / W_o / W_down k-group partials ([S][rows][width]
  // f32), added by the kernel that consumes the projection (the attention,
  // the RMSNorms)
  void* parts = nullptr;
  uint64_t parts_bytes = 0;
  // a prefill's W_down k-split partials ([2][rows][d] f32), added by the norm
  // that consumes them; grown on first use
  void* pf_parts = nullptr;
  uint64_t pf_parts_bytes = 0;
  // the generate loop's deferred LM-head argmax: per-column-block summaries
  // ([max_batch][ceil(vocab / 128)][4] u32) composed by the next step
  void* arg_sums = nullptr;
  void* lens_table = nullptr;  // [(max_len + 1)][max_batch] u32
  std::vector<void*> w_qkv, w_o, w_gu, w_down, kc, vc;
  // activations (capacity rows_cap rows) and per-sequence buffers
  uint64_t rows_cap = 0;
  void* act[CATENA_DEC_TENSOR_COUNT] = {};
  void* final_rows = nullptr;  // [max_batch] u32: index of each sequence's last row
  void* cur_tok = nullptr;     // [max_batch] u32: next input token per sequence
  // pinned host staging of final_rows; rows_copied marks the end of the last
  // copy out of it, so it is not rewritten while a copy may still read it
  uint32_t* rows_host = nullptr;
  hipEvent_t rows_copied = nullptr;
  bool rows_pending = false;
  uint32_t batch = 0, cur_len = 0, last_rows = 0;
};

namespace {

uint64_t kv_elems(const catena_decoder& m) {
  return (uint64_t)m.cfg.max_batch * m.cfg.n_heads * m.cfg.max_len * m.cfg.head_dim;
}

// bytes per row of each activation tensor
uint64_t act_row_bytes(const catena_decoder& m, int which) {
  switch (which) {
    case CATENA_DEC_X: case CATENA_DEC_ATTN_PROJ: case CATENA_DEC_H: case CATENA_DEC_FFN_OUT:
      return m.d * 4;
    case CATENA_DEC_XN: case CATENA_DEC_Q: case CATENA_DEC_ATTN: case CATENA_DEC_HN:
      return m.d * 2;
    case CATENA_DEC_QKV: return 3 * m.d * 4;
    case CATENA_DEC_GU: return 2 * m.f * 4;
    case CATENA_DEC_ACT: return m.f * 2;
    default: return 0;
  }
}

// per-batch-row tensors, sized for max_batch
uint64_t batch_tensor_bytes(const catena_decoder& m, int which) {
  switch (which) {
    case CATENA_DEC_FINAL_H: return m.cfg.max_batch * m.d * 4;
    case CATENA_DEC_FINAL_XN: return m.cfg.max_batch * m.d * 2;
    case CATENA_DEC_LOGITS: return (uint64_t)m.cfg.max_batch * m.cfg.vocab * 4;
    default: return 0;
  }
}

int alloc(uint64_t bytes, void** p) { return pool_alloc(bytes, p); }

int ensure_rows(catena_decoder& m, uint64_t rows) {
  if (rows <= m.rows_cap) return CATENA_OK;
  // queued kernels may still use the old buffers
  int st = hip_check(hipStreamSynchronize(device().stream), "hipStreamSynchronize");
  if (st) return st;
  for (int w = CATENA_DEC_X; w <= CATENA_DEC_FFN_OUT; ++w) {
    pool_free(m.act[w]);
    m.act[w] = nullptr;
  }
  m.rows_cap = 0;
  for (int w = CATENA_DEC_X; w <= CATENA_DEC_FFN_OUT; ++w) {
    st = alloc(rows * act_row_bytes(m, w), &m.act[w]);
    if (st) return st;
  }
  m.rows_cap = rows;
  return CATENA_OK;
}

void release(catena_decoder* m) {
  pool_free(m->embed);
  pool_free(m->embed_norm);
  pool_free(m->w_lm);
  pool_free(m->inv_freq);
  pool_free(m->rope_tab);
  pool_free(m->parts);
  pool_free(m->pf_parts);
  pool_free(m->arg_sums);
  pool_free(m->lens_table);
  for (auto* v : {&m->w_qkv, &m->w_o, &m->w_gu, &m->w_down, &m->kc, &m->vc})
    for (void* p : *v) pool_free(p);
  for (void*& p : m->act) {
    if (p) pool_free(p);
    p = nullptr;
  }
  pool_free(m->final_rows);
  pool_free(m->cur_tok);
  if (m->rows_copied) hipEventDestroy(m->rows_copied);
  m->rows_copied = nullptr;
  if (m->rows_host) hipHostFree(m->rows_host);
  m->rows_host = nullptr;
}

#define TRY(expr)              \
  do {                         \
    int st_ = (expr);          \
    if (st_) return st_;       \
  } while (0)

// One forward pass over rows = batch * tq tokens (tq per sequence), caches
// already holding the earlier positions; lens = positions after the append
// (every sequence at the same length len, a row of the lens table);
// final_rows selects each sequence's last row (NULL when tq == 1); next
// receives the greedy tokens.  A decode step (tq == 1, batch <= 16) runs the
// projections on the decode-shape GEMM with fused epilogues: RoPE and the
// cache append after W_qkv, the SwiGLU gate after W_gu, greedy argmax after
// W_lm; the embedding gather is fused into the first RMSNorm in both cases.
int forward(catena_decoder& m, const uint32_t* tokens, uint32_t batch, uint32_t tq,
            const uint32_t* lens, uint32_t len, const uint32_t* final_rows, uint32_t* next,
            const uint32_t* in_sums = nullptr, bool defer_argmax = false) {
  const catena_decoder_config_t& c = m.cfg;
  const uint64_t rows = (uint64_t)batch * tq, d = m.d, f = m.f;
  TRY(ensure_rows(m, rows));
  auto A = [&](int w) { return m.act[w]; };
  float* X = static_cast<float*>(A(CATENA_DEC_X));
  uint16_t* XN = static_cast<uint16_t*>(A(CATENA_DEC_XN));
  float* QKV = static_cast<float*>(A(CATENA_DEC_QKV));
  uint16_t* Q = static_cast<uint16_t*>(A(CATENA_DEC_Q));
  uint16_t* ATT = static_cast<uint16_t*>(A(CATENA_DEC_ATTN));
  float* AP = static_cast<float*>(A(CATENA_DEC_ATTN_PROJ));
  float* H = static_cast<float*>(A(CATENA_DEC_H));
  uint16_t* HN = static_cast<uint16_t*>(A(CATENA_DEC_HN));
  float* GU = static_cast<float*>(A(CATENA_DEC_GU));
  uint16_t* ACT = static_cast<uint16_t*>(A(CATENA_DEC_ACT));
  float* FO = static_cast<float*>(A(CATENA_DEC_FFN_OUT));
  const float scale = (float)(1.0 / std::sqrt((double)c.head_dim));
  const float* inv = static_cast<const float*>(m.inv_freq);
  const bool step = tq == 1 && batch <= 16;
  const uint16_t* embed = static_cast<const uint16_t*>(m.embed);
  if (m.embed_norm_stale) {
    TRY(embed_norm_table_bf16(embed, c.vocab, static_cast<uint16_t*>(m.embed_norm), d));
    m.embed_norm_stale = false;
  }

  uint32_t parts_down = 0;  // k groups of the last W_down partials (decode step)
  // a prefill's W_down as two k-half partials on 256 x 256 tiles (the whole
  // chip at C5, where one pass fills half of it with those tiles): the norm
  // that consumes them adds P0 + P1 and writes the sum to FO for its rows
  const uint32_t kPfSplits = 2;
  const bool down_split = !step && (uint64_t)(rows / 256) * (d / 256) <= 128 &&
                          gemm_bf16_ksplit_fits(rows, d, f, kPfSplits, A(CATENA_DEC_ACT), m.w_down[0],
                                                A(CATENA_DEC_ACT));
  if (down_split && m.pf_parts_bytes < kPfSplits * rows * d * 4) {
    TRY(hip_check(hipStreamSynchronize(device().stream), "hipStreamSynchronize"));
    pool_free(m.pf_parts);
    m.pf_parts = nullptr;
    m.pf_parts_bytes = 0;
    TRY(alloc(kPfSplits * rows * d * 4, &m.pf_parts));
    m.pf_parts_bytes = kPfSplits * rows * d * 4;
  }
  float* PF = static_cast<float*>(m.pf_parts);
  // a decode step whose attention is the eight-wave kernel takes q / k / v
  // as W_qkv's partials
  const bool few_attn = step && attn_few_fits(batch, 1, c.n_heads, c.max_len);
  for (uint32_t l = 0; l < c.n_layers; ++l) {
    // x_l = h_{l-1} + ffn_{l-1} (layer 0: the embedding), xn = bf16(rmsnorm(x_l)).
    // A decode step's layer 0 reads xn as rows of the normalized embedding
    // table (the same kernel's bits, computed once per embedding) and x as
    // the embedding rows themselves: no norm runs for it.
    const bool gathered = step && l == 0;
    if (l == 0 && !gathered)
      TRY(embed_rmsnorm_bf16(tokens, embed, c.vocab, X, XN, rows, d));
    else if (l > 0 && step)
      // the previous layer's W_down arrives as k-group partials
      TRY(residual_parts_rmsnorm_bf16(H, static_cast<const float*>(m.parts), parts_down, FO, nullptr,
                                      X, XN, rows, rows, d));
    else if (l > 0 && down_split)
      TRY(residual_parts_rmsnorm_bf16(H, PF, kPfSplits, FO, nullptr, X, XN, rows, rows, d));
    else if (l > 0)
      TRY(catena_mi355x_residual_rmsnorm_bf16(H, FO, nullptr, X, XN, rows, d));
    uint16_t* kc = static_cast<uint16_t*>(m.kc[l]);
    uint16_t* vc = static_cast<uint16_t*>(m.vc[l]);
    const uint16_t* wqkv = static_cast<const uint16_t*>(m.w_qkv[l]);
    if (step) {
      DecodeEpiArgs e;
      e.q_out = Q;
      e.k_cache = kc;
      e.v_cache = vc;
      e.lens = lens;
      e.inv_freq = inv;
      e.rope_tab = static_cast<const float*>(m.rope_tab);
      e.heads = c.n_heads;
      e.max_len = c.max_len;
      const uint16_t* xn = XN;
      if (gathered) {
        xn = static_cast<const uint16_t*>(m.embed_norm);
        e.x_rows_limit = c.vocab;
        if (in_sums) {
          // the tokens are the previous step's deferred argmax: composed
          // here from its summaries and written to `tokens` for the norm
          e.x_sums = in_sums;
          e.x_sums_blocks = (uint32_t)((c.vocab + 127) / 128);
          e.x_sums_cols = c.vocab;
          e.x_rows_out = const_cast<uint32_t*>(tokens);
        } else {
          e.x_rows = tokens;
        }
      }
      if (few_attn) {
        // W_qkv as k-group partials: the attention adds them, rotates q and
        // k and appends the caches itself (no hand-off in the projection)
        uint32_t parts_qkv = 0;
        float* P = static_cast<float*>(m.parts);
        TRY(gemm_bf16_decode_parts(xn, wqkv, P, m.parts_bytes, rows, 3 * d, d, &parts_qkv, e));
        FewQkvArgs fq;
        fq.parts = P;
        fq.part_stride = rows * 3 * d;
        fq.n_parts = parts_qkv;
        fq.rope_tab = static_cast<const float*>(m.rope_tab);
        fq.q_out = Q;
        fq.qkv_out = QKV;
        fq.k_cache = kc;
        fq.v_cache = vc;
        const int st_ = attn_few_launch(nullptr, kc, vc, lens, ATT, batch, 1, c.n_heads, c.max_len, scale,
                                        false, fq);
        if (st_ < 0) return fail(CATENA_ERR_UNSUPPORTED, "eight-wave attention did not apply");
        TRY(st_);
      } else {
        TRY(gemm_bf16_decode(xn, wqkv, QKV, rows, 3 * d, d, DecodeEpilogue::Rope, e));
      }
    } else if (gemm_bf16_rope_fits(rows, d, tq, c.n_heads, XN, wqkv, Q, kc, vc, m.rope_tab)) {
      // RoPE, bf16 q and the cache append in the projection's epilogue: the
      // f32 product (3d floats per row) is never written
      TRY(gemm_bf16_rope_qkv(XN, wqkv, static_cast<const float*>(m.rope_tab), lens, Q, kc, vc, rows, d,
                             tq, c.n_heads, c.max_len));
    } else {
      TRY(catena_mi355x_gemm_bf16(XN, wqkv, QKV, rows, 3 * d, d, 1));
      TRY(catena_mi355x_rope_qkv_bf16(QKV, inv, lens, Q, kc, vc, batch, tq, c.n_heads, c.head_dim,
                                      c.max_len));
    }
    if (!(step && few_attn))
      TRY(attn_causal(Q, kc, vc, lens, ATT, batch, tq, c.n_heads, c.max_len, len, c.head_dim, scale,
                      0));
    if (step) {
      // W_o without its split-K hand-off: the norm below adds the k-group
      // partials (and writes their sum to AP)
      uint32_t parts_o = 0;
      float* P = static_cast<float*>(m.parts);
      TRY(gemm_bf16_decode_parts(ATT, static_cast<const uint16_t*>(m.w_o[l]), P, m.parts_bytes, rows, d,
                                 d, &parts_o));
      if (gathered)
        TRY(embed_residual_rmsnorm_bf16(tokens, embed, c.vocab, P, H, HN, rows, d, parts_o, AP));
      else
        TRY(residual_parts_rmsnorm_bf16(X, P, parts_o, AP, nullptr, H, HN, rows, rows, d));
    } else {
      TRY(catena_mi355x_gemm_bf16(ATT, static_cast<const uint16_t*>(m.w_o[l]), AP, rows, d, d, 1));
      TRY(catena_mi355x_residual_rmsnorm_bf16(X, AP, nullptr, H, HN, rows, d));
    }
    const uint16_t* wgu = static_cast<const uint16_t*>(m.w_gu[l]);
    if (step) {
      DecodeEpiArgs e;
      e.act = ACT;
      // whole K per workgroup: the block weights stay in the Infinity Cache
      // from step to step (the LM head streams past it), and for this
      // projection one pass without the split-K hand-off is the faster
      // form there (measured in the C5 step: 2.6 us less than two k groups)
      TRY(gemm_bf16_decode(HN, wgu, GU, rows, 2 * f, d, DecodeEpilogue::Silu, e, nullptr, 0,
                           true));
    } else if (gemm_bf16_silu_fits(rows, 2 * f, d, HN, wgu, ACT)) {
      // the SwiGLU gate in the GEMM's epilogue: the f32 gate / up product
      // (4x the bytes of act) is never written
      TRY(catena_mi355x_gemm_bf16_silu(HN, wgu, ACT, rows, 2 * f, d));
    } else {
      TRY(catena_mi355x_gemm_bf16(HN, wgu, GU, rows, 2 * f, d, 1));
      TRY(catena_mi355x_silu_mul_bf16(GU, ACT, rows, (uint32_t)f, 64));
    }
    if (step)
      // k-group partials, added by the next norm (the next layer's input
      // norm or the final norm)
      TRY(gemm_bf16_decode_parts(ACT, static_cast<const uint16_t*>(m.w_down[l]), static_cast<float*>(m.parts),
                                 m.parts_bytes, rows, d, f, &parts_down));
    else if (down_split)
      TRY(gemm_bf16_f32_ksplit(ACT, static_cast<const uint16_t*>(m.w_down[l]), PF, rows, d, f, kPfSplits));
    else
      TRY(catena_mi355x_gemm_bf16(ACT, static_cast<const uint16_t*>(m.w_down[l]), FO, rows, d, f, 1));
  }
  float* FH = static_cast<float*>(A(CATENA_DEC_FINAL_H));
  uint16_t* FXN = static_cast<uint16_t*>(A(CATENA_DEC_FINAL_XN));
  float* LG = static_cast<float*>(A(CATENA_DEC_LOGITS));
  if (step)
    TRY(residual_parts_rmsnorm_bf16(H, static_cast<const float*>(m.parts), parts_down, FO, final_rows, FH,
                                    FXN, batch, rows, d));
  else if (down_split)
    TRY(residual_parts_rmsnorm_bf16(H, PF, kPfSplits, FO, final_rows, FH, FXN, batch, rows, d));
  else
    TRY(catena_mi355x_residual_rmsnorm_bf16(H, FO, final_rows, FH, FXN, batch, d));
  const uint16_t* wlm = static_cast<const uint16_t*>(m.w_lm);
  if (batch <= 16) {
    DecodeEpiArgs e;
    if (defer_argmax) {
      // logits and column-block summaries only; the next step's W_qkv (or
      // argmax_compose after the last step) composes the argmax
      e.arg_defer = 1;
      e.arg_partials = static_cast<uint32_t*>(m.arg_sums);
    } else {
      e.idx = next;
    }
    TRY(gemm_bf16_decode(FXN, wlm, LG, batch, c.vocab, d, DecodeEpilogue::Argmax, e));
  } else {
    TRY(catena_mi355x_gemm_bf16(FXN, wlm, LG, batch, c.vocab, d, 1));
    TRY(catena_mi355x_argmax_f32(LG, next, batch, c.vocab));
  }
  return CATENA_OK;
}

}  // namespace

extern "C" {

int catena_mi355x_decoder_create(const catena_decoder_config_t* cfg, catena_decoder_t** out) {
  if (!out || !cfg) return fail(CATENA_ERR_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  int st = ensure_init();
  if (st) return st;
  const catena_decoder_config_t& c = *cfg;
  if (c.head_dim != 128) return fail(CATENA_ERR_UNSUPPORTED, "decoder head_dim must be 128");
  if (c.n_heads == 0 || c.n_layers == 0 || c.vocab == 0 || c.max_batch == 0 || c.max_len == 0 ||
      c.ffn_dim == 0)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "decoder sizes must be non-zero");
  if ((uint64_t)c.n_heads * c.head_dim != c.d_model)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "d_model must equal n_heads * head_dim");
  if (c.ffn_dim % 64 != 0 || c.vocab % 8 != 0)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "ffn_dim must be a multiple of 64, vocab of 8");
  if (!(c.rope_base > 1.0f)) return fail(CATENA_ERR_INVALID_ARGUMENT, "rope_base must exceed 1");
  // sizes the kernels and tables can hold: the attention keeps one f32 score
  // per cache position in LDS; the uniform-length lens table has
  // (max_len + 1) x max_batch entries; every byte count below fits 64 bits
  const size_t attn_lds = attn_lds_bytes(c.max_len);
  if (attn_lds > device().max_lds)
    return fail(CATENA_ERR_UNSUPPORTED, "max_len %u exceeds the attention's LDS (%zu B > %zu B)",
                c.max_len, attn_lds, device().max_lds);
  // every RMSNorm holds a row of d_model values (and their squares) in LDS
  const size_t norm_lds = rmsnorm_lds_bytes(c.d_model);
  if (norm_lds > device().max_lds)
    return fail(CATENA_ERR_UNSUPPORTED, "d_model %u exceeds the RMSNorm's LDS (%zu B > %zu B)",
                c.d_model, norm_lds, device().max_lds);
  if (c.max_batch > 4096 || c.n_heads > 4096 || c.n_layers > 4096 || c.ffn_dim > (1u << 24) ||
      c.vocab > (1u << 26))
    return fail(CATENA_ERR_UNSUPPORTED,
                "decoder config beyond the supported sizes (max_batch, n_heads, n_layers <= 4096; "
                "ffn_dim <= 2^24; vocab <= 2^26)");

  catena_decoder* m = new (std::nothrow) catena_decoder();
  if (!m) return fail(CATENA_ERR_OUT_OF_MEMORY, "decoder allocation");
  m->cfg = c;
  m->d = c.d_model;
  m->f = c.ffn_dim;
  const uint64_t d = m->d, f = m->f;
  auto fail_out = [&](int s) {
    release(m);
    delete m;
    return s;
  };
  if ((st = alloc((uint64_t)c.vocab * d * 2, &m->embed))) return fail_out(st);
  if ((st = alloc(((uint64_t)c.vocab + 1) * d * 2, &m->embed_norm))) return fail_out(st);
  if ((st = alloc(d * c.vocab * 2, &m->w_lm))) return fail_out(st);
  try {
    for (auto* v : {&m->w_qkv, &m->w_o, &m->w_gu, &m->w_down, &m->kc, &m->vc}) v->reserve(c.n_layers);
  } catch (const std::bad_alloc&) {
    return fail_out(fail(CATENA_ERR_OUT_OF_MEMORY, "decoder layer tables"));
  }
  for (uint32_t l = 0; l < c.n_layers; ++l) {
    void *a = nullptr, *b = nullptr, *g = nullptr, *dn = nullptr, *k = nullptr, *v = nullptr;
    if ((st = alloc(d * 3 * d * 2, &a))) return fail_out(st);
    m->w_qkv.push_back(a);
    if ((st = alloc(d * d * 2, &b))) return fail_out(st);
    m->w_o.push_back(b);
    if ((st = alloc(d * 2 * f * 2, &g))) return fail_out(st);
    m->w_gu.push_back(g);
    if ((st = alloc(f * d * 2, &dn))) return fail_out(st);
    m->w_down.push_back(dn);
    if ((st = alloc(kv_elems(*m) * 2, &k))) return fail_out(st);
    m->kc.push_back(k);
    if ((st = alloc(kv_elems(*m) * 2, &v))) return fail_out(st);
    m->vc.push_back(v);
  }
  for (int w = CATENA_DEC_FINAL_H; w <= CATENA_DEC_LOGITS; ++w)
    if ((st = alloc(batch_tensor_bytes(*m, w), &m->act[w]))) return fail_out(st);
  if ((st = alloc(c.max_batch * 4, &m->act[CATENA_DEC_LENS]))) return fail_out(st);
  if ((st = alloc(c.max_batch * 4, &m->final_rows))) return fail_out(st);
  if ((st = alloc(c.max_batch * 4, &m->cur_tok))) return fail_out(st);
  if ((st = hip_check(hipHostMalloc(reinterpret_cast<void**>(&m->rows_host), c.max_batch * 4),
                      "hipHostMalloc(final rows)")))
    return fail_out(st);
  if ((st = hip_check(hipEventCreateWithFlags(&m->rows_copied, hipEventDisableTiming),
                      "hipEventCreate(final rows)")))
    return fail_out(st);

  // host-computed tables: RoPE frequencies and the uniform-length lens rows
  std::vector<float> inv;
  std::vector<uint32_t> lt;
  try {
    inv.resize(c.head_dim / 2);
    lt.resize((uint64_t)(c.max_len + 1) * c.max_batch);
  } catch (const std::bad_alloc&) {
    return fail_out(fail(CATENA_ERR_OUT_OF_MEMORY, "host tables of the decoder"));
  }
  if ((st = catena_mi355x_rope_inv_freq(inv.data(), c.head_dim, (double)c.rope_base)))
    return fail_out(st);
  if ((st = alloc(inv.size() * 4, &m->inv_freq))) return fail_out(st);
  for (uint64_t t = 0; t <= c.max_len; ++t)
    for (uint32_t b = 0; b < c.max_batch; ++b) lt[t * c.max_batch + b] = (uint32_t)t;
  if ((st = alloc(lt.size() * 4, &m->lens_table))) return fail_out(st);
  if ((st = catena_mem_write(catena_mem_t{m->inv_freq, inv.size() * 4}, 0, inv.data(), inv.size() * 4)))
    return fail_out(st);
  // the decode step's RoPE reads its rotations from a table of every
  // position (computed by the same functions, so the same bits)
  if ((st = alloc((uint64_t)c.max_len * c.head_dim * 4, &m->rope_tab))) return fail_out(st);
  if ((st = rope_table_f32(static_cast<const float*>(m->inv_freq), static_cast<float*>(m->rope_tab),
                           c.max_len, c.head_dim / 2)))
    return fail_out(st);
  if ((st = catena_mem_write(catena_mem_t{m->lens_table, lt.size() * 4}, 0, lt.data(), lt.size() * 4)))
    return fail_out(st);
  // partials of the decode step's two row-reduced projections: S k groups of
  // max_batch x d floats for W_o (k = d) and W_down (k = d_ff)
  {
    uint32_t s_o = 0, s_down = 0, s_qkv = 0;
    decode_partials_bytes(c.max_batch, c.d_model, c.d_model, &s_o);
    decode_partials_bytes(c.max_batch, c.d_model, c.ffn_dim, &s_down);
    decode_partials_bytes(c.max_batch, 3ull * c.d_model, c.d_model, &s_qkv);
    const uint64_t groups = std::max<uint64_t>(1, std::max(s_o, s_down));
    m->parts_bytes = std::max<uint64_t>(groups * c.d_model, std::max<uint64_t>(1, s_qkv) * 3ull * c.d_model) *
                     c.max_batch * 4;
    if ((st = alloc(m->parts_bytes, &m->parts))) return fail_out(st);
  }
  if ((st = alloc((uint64_t)c.max_batch * ((c.vocab + 127) / 128) * 16, &m->arg_sums))) return fail_out(st);
  *out = m;
  return CATENA_OK;
}

void catena_mi355x_decoder_destroy(catena_decoder_t* dec) {
  if (!dec) return;
  hipStreamSynchronize(device().stream);
  release(dec);
  delete dec;
}

int catena_mi355x_decoder_tensor(catena_decoder_t* dec, uint32_t which, uint32_t layer,
                                 catena_mem_t* out) {
  if (!dec || !out) return fail(CATENA_ERR_INVALID_ARGUMENT, "null argument");
  catena_decoder& m = *dec;
  const catena_decoder_config_t& c = m.cfg;
  const bool per_layer = which == CATENA_DEC_W_QKV || which == CATENA_DEC_W_O ||
                         which == CATENA_DEC_W_GU || which == CATENA_DEC_W_DOWN ||
                         which == CATENA_DEC_K_CACHE || which == CATENA_DEC_V_CACHE;
  if (per_layer && layer >= c.n_layers)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "layer %u out of range", layer);
  const uint64_t d = m.d, f = m.f;
  switch (which) {
    case CATENA_DEC_EMBED:
      // the caller may write the embedding through this: rebuild its
      // normalized table before the next forward
      *out = {m.embed, (uint64_t)c.vocab * d * 2};
      m.embed_norm_stale = true;
      m.embed_exposed = true;
      break;
    case CATENA_DEC_EMBED_NORM: *out = {m.embed_norm, ((uint64_t)c.vocab + 1) * d * 2}; break;
    case CATENA_DEC_W_QKV: *out = {m.w_qkv[layer], d * 3 * d * 2}; break;
    case CATENA_DEC_W_O: *out = {m.w_o[layer], d * d * 2}; break;
    case CATENA_DEC_W_GU: *out = {m.w_gu[layer], d * 2 * f * 2}; break;
    case CATENA_DEC_W_DOWN: *out = {m.w_down[layer], f * d * 2}; break;
    case CATENA_DEC_W_LM: *out = {m.w_lm, d * c.vocab * 2}; break;
    case CATENA_DEC_K_CACHE: *out = {m.kc[layer], kv_elems(m) * 2}; break;
    case CATENA_DEC_V_CACHE: *out = {m.vc[layer], kv_elems(m) * 2}; break;
    case CATENA_DEC_INV_FREQ: *out = {m.inv_freq, (uint64_t)c.head_dim / 2 * 4}; break;
    case CATENA_DEC_FINAL_H: case CATENA_DEC_FINAL_XN: case CATENA_DEC_LOGITS:
      *out = {m.act[which], batch_tensor_bytes(m, (int)which) / c.max_batch * m.batch};
      break;
    case CATENA_DEC_LENS: *out = {m.act[which], (uint64_t)m.batch * 4}; break;
    default:
      if (which >= CATENA_DEC_X && which <= CATENA_DEC_FFN_OUT) {
        *out = {m.act[which], m.act[which] ? m.last_rows * act_row_bytes(m, (int)which) : 0};
        break;
      }
      return fail(CATENA_ERR_INVALID_ARGUMENT, "unknown decoder tensor %u", which);
  }
  return CATENA_OK;
}

int catena_mi355x_decoder_init_weights(catena_decoder_t* dec, uint64_t seed, float std) {
  if (!dec) return fail(CATENA_ERR_INVALID_ARGUMENT, "null decoder");
  catena_decoder& m = *dec;
  const uint64_t d = m.d, f = m.f, V = m.cfg.vocab;
  TRY(catena_mi355x_fill_normal_bf16(static_cast<uint16_t*>(m.embed), V * d, seed, 0, std));
  TRY(catena_mi355x_fill_normal_bf16(static_cast<uint16_t*>(m.w_lm), d * V, seed, 1, std));
  for (uint32_t l = 0; l < m.cfg.n_layers; ++l) {
    const uint64_t s = 16 + 4ull * l;
    TRY(catena_mi355x_fill_normal_bf16(static_cast<uint16_t*>(m.w_qkv[l]), d * 3 * d, seed, s, std));
    TRY(catena_mi355x_fill_normal_bf16(static_cast<uint16_t*>(m.w_o[l]), d * d, seed, s + 1, std));
    TRY(catena_mi355x_fill_normal_bf16(static_cast<uint16_t*>(m.w_gu[l]), d * 2 * f, seed, s + 2, std));
    TRY(catena_mi355x_fill_normal_bf16(static_cast<uint16_t*>(m.w_down[l]), f * d, seed, s + 3, std));
  }
  TRY(embed_norm_table_bf16(static_cast<const uint16_t*>(m.embed), (uint32_t)V,
                            static_cast<uint16_t*>(m.embed_norm), d));
  m.embed_norm_stale = false;
  return CATENA_OK;
}

int catena_mi355x_decoder_prefill(catena_decoder_t* dec, const uint32_t* tokens, uint32_t batch,
                                  uint32_t t, uint32_t* next) {
  if (!dec || !tokens || !next) return fail(CATENA_ERR_INVALID_ARGUMENT, "null argument");
  catena_decoder& m = *dec;
  const catena_decoder_config_t& c = m.cfg;
  if (batch == 0 || batch > c.max_batch)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "batch %u outside 1..%u", batch, c.max_batch);
  if (t == 0 || t > c.max_len)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "prefill length %u outside 1..%u", t, c.max_len);
  Device& dv = device();
  if (m.embed_exposed) m.embed_norm_stale = true;
  // the staging buffer is pinned, so the copy below reads it when the stream
  // reaches it: wait for the previous prefill's copy before rewriting it
  if (m.rows_pending) TRY(hip_check(hipEventSynchronize(m.rows_copied), "hipEventSynchronize"));
  for (uint32_t b = 0; b < batch; ++b) m.rows_host[b] = b * t + (t - 1);
  TRY(hip_check(hipMemcpyAsync(m.final_rows, m.rows_host, batch * 4, hipMemcpyHostToDevice,
                               dv.stream),
                "hipMemcpyAsync(final rows)"));
  TRY(hip_check(hipEventRecord(m.rows_copied, dv.stream), "hipEventRecord(final rows)"));
  m.rows_pending = true;
  const uint32_t* lens = static_cast<const uint32_t*>(m.lens_table) + (uint64_t)t * c.max_batch;
  m.batch = batch;
  m.last_rows = batch * t;
  TRY(forward(m, tokens, batch, t, lens, t, static_cast<const uint32_t*>(m.final_rows),
              static_cast<uint32_t*>(m.cur_tok)));
  m.cur_len = t;
  TRY(hip_check(hipMemcpyAsync(m.act[CATENA_DEC_LENS], lens, batch * 4, hipMemcpyDeviceToDevice,
                               dv.stream),
                "hipMemcpyAsync(lens)"));
  return hip_check(hipMemcpyAsync(next, m.cur_tok, batch * 4, hipMemcpyDeviceToDevice, dv.stream),
                   "hipMemcpyAsync(next)");
}

int catena_mi355x_decoder_generate(catena_decoder_t* dec, uint32_t steps, uint32_t* out) {
  if (!dec || (steps > 0 && !out)) return fail(CATENA_ERR_INVALID_ARGUMENT, "null argument");
  catena_decoder& m = *dec;
  const catena_decoder_config_t& c = m.cfg;
  if (m.batch == 0) return fail(CATENA_ERR_INVALID_ARGUMENT, "generate before prefill");
  if ((uint64_t)m.cur_len + steps > c.max_len)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "%u steps after %u positions overflow the %u-position cache",
                steps, m.cur_len, c.max_len);
  if (steps == 0) return CATENA_OK;
  if (m.embed_exposed) m.embed_norm_stale = true;
  const uint32_t B = m.batch;
  // Each step's argmax is composed by the next step's first GEMM, from the
  // LM head's column-block summaries (the LM head then ends without its
  // completion ticket); the last step's by argmax_compose.  Decode steps
  // whose first GEMM streams (d % 32 == 0) and whose LM head is the decode
  // GEMM (batch <= 16) only.
  const bool defer = B <= 16 && m.d % 32 == 0;
  const uint32_t* sums = static_cast<const uint32_t*>(m.arg_sums);
  for (uint32_t s = 0; s < steps; ++s) {
    const uint32_t* in = s == 0 ? static_cast<const uint32_t*>(m.cur_tok) : out + (uint64_t)(s - 1) * B;
    const uint32_t* lens =
        static_cast<const uint32_t*>(m.lens_table) + (uint64_t)(m.cur_len + 1) * c.max_batch;
    m.last_rows = B;
    TRY(forward(m, in, B, 1, lens, m.cur_len + 1, nullptr, out + (uint64_t)s * B,
                defer && s > 0 ? sums : nullptr, defer));
    m.cur_len += 1;
  }
  if (defer)
    TRY(argmax_compose(sums, B, (uint32_t)((c.vocab + 127) / 128), c.vocab, out + (uint64_t)(steps - 1) * B));
  Device& dv = device();
  const uint32_t* lens = static_cast<const uint32_t*>(m.lens_table) + (uint64_t)m.cur_len * c.max_batch;
  TRY(hip_check(hipMemcpyAsync(m.act[CATENA_DEC_LENS], lens, B * 4, hipMemcpyDeviceToDevice, dv.stream),
                "hipMemcpyAsync(lens)"));
  return hip_check(hipMemcpyAsync(m.cur_tok, out + (uint64_t)(steps - 1) * B, B * 4,
                                  hipMemcpyDeviceToDevice, dv.stream),
                   "hipMemcpyAsync(cur_tok)");
}

}  // extern "C"
