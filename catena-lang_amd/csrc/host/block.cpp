// Kernel ABI of the decoder-block pieces (block.hip, causal attention) and
// the program ABI of the two stdlib ops they mirror (nn.rmsnorm,
// tensor.argmax-f32).
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>

#include "internal.h"

using namespace catena;

namespace {
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

int rmsnorm_launch(const float* x, const float* resid, const uint32_t* row_index, float* h_out,
                   float* y_f32, uint16_t* y_bf16, uint64_t rows, uint64_t n,
                   const uint32_t* tokens = nullptr, const uint16_t* table = nullptr,
                   uint32_t vocab = 0, uint32_t resid_parts = 1, uint64_t resid_stride = 0,
                   float* resid_out = nullptr) {
  int st = ensure_init();
  if (st) return st;
  if (rows == 0 || n == 0) return CATENA_OK;
  // input rows: x, or the embedding gather (tokens into table), or the
  // table's own rows (neither x nor tokens)
  if ((!x && !table) || (!y_f32 && !y_bf16)) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if ((tokens || !x) && (!table || (n % 4 == 0 && (reinterpret_cast<uintptr_t>(table) & 7u))))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "embedding table missing or misaligned");
  if (rows > 0x7FFFFFFFull || n > 0xFFFFFFFFull)
    return fail(CATENA_ERR_UNSUPPORTED, "rmsnorm shape too large");
  if (n % 4 == 0) {
    const void* ptrs[] = {x, resid, h_out, y_f32, resid_out};
    for (const void* p : ptrs)
      if (p && !aligned16(p))
        return fail(CATENA_ERR_INVALID_ARGUMENT, "rmsnorm rows must be 16-byte aligned");
    if (y_bf16 && (reinterpret_cast<uintptr_t>(y_bf16) & 7u))
      return fail(CATENA_ERR_INVALID_ARGUMENT, "rmsnorm bf16 output must be 8-byte aligned");
  }
  const uint64_t n_pad = (n + 3) & ~3ull;
  const size_t lds = 2 * n_pad * sizeof(float);  // dynamic part
  if (rmsnorm_lds_bytes(n) > device().max_lds)
    return fail(CATENA_ERR_UNSUPPORTED, "rmsnorm row of %llu needs %zu B of LDS",
                (unsigned long long)n, rmsnorm_lds_bytes(n));
  if (resid_parts == 0 || (resid_parts > 1 && (!resid || (n % 4 == 0 && resid_stride % 4 != 0))))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "rmsnorm residual partials");
  uint32_t n32 = (uint32_t)n;
  void* args[] = {&x,      &resid, &row_index, &h_out,       &y_f32,       &y_bf16,   &n32,
                  &tokens, &table, &vocab,     &resid_parts, &resid_stride, &resid_out};
  return launch(KernelId::RmsnormRows, dim3((unsigned)rows), dim3(256), lds, args);
}
}  // namespace

namespace catena {
int embed_rmsnorm_bf16(const uint32_t* tokens, const uint16_t* table, uint32_t vocab,
                       float* x_out, uint16_t* y, uint64_t rows, uint64_t n) {
  if (!tokens || !y) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  return rmsnorm_launch(nullptr, nullptr, nullptr, x_out, nullptr, y, rows, n, tokens, table, vocab);
}

int embed_residual_rmsnorm_bf16(const uint32_t* tokens, const uint16_t* table, uint32_t vocab,
                                const float* resid, float* h_out, uint16_t* y, uint64_t rows,
                                uint64_t n, uint32_t resid_parts, float* resid_out) {
  if (!tokens || !resid || !y) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  return rmsnorm_launch(nullptr, resid, nullptr, h_out, nullptr, y, rows, n, tokens, table, vocab,
                        resid_parts, rows * n, resid_out);
}

int residual_parts_rmsnorm_bf16(const float* x, const float* resid, uint32_t resid_parts,
                                float* resid_out, const uint32_t* row_index, float* h_out,
                                uint16_t* y, uint64_t rows, uint64_t resid_rows, uint64_t n) {
  if (!x || !resid || !y) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  return rmsnorm_launch(x, resid, row_index, h_out, nullptr, y, rows, n, nullptr, nullptr, 0,
                        resid_parts, resid_rows * n, resid_out);
}

int embed_norm_table_bf16(const uint16_t* table, uint32_t vocab, uint16_t* y, uint64_t n) {
  if (!table || !y) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  return rmsnorm_launch(nullptr, nullptr, nullptr, nullptr, nullptr, y, (uint64_t)vocab + 1, n, nullptr,
                        table, vocab);
}

int rope_table_f32(const float* inv_freq, float* tab, uint32_t positions, uint32_t half) {
  int st = ensure_init();
  if (st) return st;
  if (!inv_freq || !tab) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (positions == 0 || half == 0) return CATENA_OK;
  if (positions > 65535) return fail(CATENA_ERR_UNSUPPORTED, "rope table of %u positions", positions);
  void* args[] = {&inv_freq, &tab, &positions, &half};
  return launch(KernelId::RopeTable, dim3((unsigned)ceil_div(half, 256), positions), dim3(256), 0, args);
}
}  // namespace catena

extern "C" {

int catena_mi355x_attn_causal_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                   const uint32_t* lens, void* o, uint32_t batch, uint32_t tq,
                                   uint32_t heads, uint32_t max_len, uint32_t head_dim,
                                   float scale, int out_f32) {
  return catena::attn_causal(q, k, v, lens, o, batch, tq, heads, max_len, max_len, head_dim, scale,
                             out_f32);
}
}  // extern "C"

namespace catena {
int attn_causal(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint32_t* lens,
                void* o, uint32_t batch, uint32_t tq, uint32_t heads, uint32_t max_len,
                uint32_t len_bound, uint32_t head_dim, float scale, int out_f32) {
  int st = ensure_init();
  if (st) return st;
  if (head_dim != 128)
    return fail(CATENA_ERR_UNSUPPORTED, "attention head_dim %u unsupported (only 128)", head_dim);
  const uint64_t blocks = (uint64_t)batch * tq * heads;
  if (blocks == 0) return CATENA_OK;
  if (!q || !lens || !o || (max_len > 0 && (!k || !v)))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (!aligned16(k) || !aligned16(v))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "K/V caches must be 16-byte aligned");
  if (blocks > 0x7FFFFFFFu) return fail(CATENA_ERR_UNSUPPORTED, "too many queries");
  // Many queries per sequence: the block-of-16-queries kernel, which reads
  // each K / V row once per block (its score buffer holds whole 64-key
  // blocks of rows up to the longest prefix, bounded by len_bound (every
  // lens[b] <= len_bound) and max_len, so it is used while two workgroups
  // still fit a CU, bound <= 1088, and four share one for bounds up to 512;
  // it reads q rows with 16-byte loads); otherwise the one-query-per-
  // workgroup kernel.  Both give the same bits.
  const uint32_t rows_bound = len_bound < max_len ? len_bound : max_len;
  const size_t lds_pf =
      16 * 136 * 2 + 3 * 16 * 4 + 3 * 4 * 16 * 4 + (size_t)ceil_div(rows_bound, 64) * 64 * 17 * 4;
  if (tq >= 8 && lds_pf <= 80 * 1024 && aligned16(q)) {
    const uint64_t nqb = ceil_div(tq, 16);
    const uint64_t grid = (uint64_t)batch * heads * nqb;
    if (grid > 0x7FFFFFFFu) return fail(CATENA_ERR_UNSUPPORTED, "too many query blocks");
    void* pargs[] = {&q, &k, &v, &lens, &o, &batch, &heads, &max_len, &tq, &scale};
    return launch(out_f32 ? KernelId::AttnPrefillD128F32 : KernelId::AttnPrefillD128Bf16,
                  dim3((unsigned)grid), dim3(256), lds_pf, pargs);
  }
  const size_t lds = attn_lds_bytes(max_len);
  if (lds > device().max_lds)
    return fail(CATENA_ERR_UNSUPPORTED, "max_len %u needs %zu B of LDS (device has %zu)", max_len,
                lds, device().max_lds);
  // few (query, head) pairs: the eight-wave kernel spreads each over a CU
  int split = attn_few_launch(q, k, v, lens, o, batch, tq, heads, max_len, scale, out_f32 != 0);
  if (split >= 0) return split;
  void* args[] = {&q, &k, &v, &lens, &o, &heads, &max_len, &tq, &scale};
  return launch(out_f32 ? KernelId::AttnCausalD128F32 : KernelId::AttnCausalD128Bf16,
                dim3((unsigned)blocks), dim3(256), lds, args);
}
}  // namespace catena

extern "C" {

int catena_mi355x_rmsnorm_f32(const float* x, float* y, uint64_t rows, uint64_t n) {
  if (x && x == y) return fail(CATENA_ERR_INVALID_ARGUMENT, "rmsnorm output may not alias input");
  return rmsnorm_launch(x, nullptr, nullptr, nullptr, y, nullptr, rows, n);
}

int catena_mi355x_residual_rmsnorm_bf16(const float* x, const float* resid,
                                        const uint32_t* row_index, float* h_out, uint16_t* y,
                                        uint64_t rows, uint64_t n) {
  if (!y) return fail(CATENA_ERR_INVALID_ARGUMENT, "null output");
  return rmsnorm_launch(x, resid, row_index, h_out, nullptr, y, rows, n);
}

int catena_mi355x_embed_bf16(const uint32_t* tokens, const uint16_t* table, float* x,
                             uint64_t rows, uint32_t vocab, uint32_t d) {
  int st = ensure_init();
  if (st) return st;
  if (rows == 0 || d == 0) return CATENA_OK;
  if (!tokens || !x || (vocab > 0 && !table)) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (d % 8 != 0 || !aligned16(table) || !aligned16(x))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "embedding needs d %% 8 == 0 and 16-byte aligned rows");
  if (rows > 65535) return fail(CATENA_ERR_UNSUPPORTED, "embedding of more than 65535 rows");
  void* args[] = {&tokens, &table, &x, &vocab, &d};
  return launch(KernelId::EmbedRowsBf16, dim3((unsigned)ceil_div(d, 2048), (unsigned)rows),
                dim3(256), 0, args);
}

int catena_mi355x_rope_inv_freq(float* out_host, uint32_t head_dim, double base) {
  if (!out_host || head_dim == 0 || head_dim % 2 != 0)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "rope needs an even head_dim and an output");
  for (uint32_t i = 0; i < head_dim / 2; ++i)
    out_host[i] = (float)(1.0 / std::pow(base, (2.0 * i) / head_dim));
  return CATENA_OK;
}

int catena_mi355x_rope_table_f32(const float* inv_freq, float* tab, uint32_t positions,
                                 uint32_t head_dim) {
  if (head_dim % 2 != 0) return fail(CATENA_ERR_INVALID_ARGUMENT, "rope needs an even head_dim");
  return rope_table_f32(inv_freq, tab, positions, head_dim / 2);
}

int catena_mi355x_rope_qkv_bf16(const float* qkv, const float* inv_freq, const uint32_t* lens,
                                uint16_t* q, uint16_t* k_cache, uint16_t* v_cache,
                                uint32_t batch, uint32_t tq, uint32_t heads, uint32_t head_dim,
                                uint32_t max_len) {
  int st = ensure_init();
  if (st) return st;
  const uint64_t rows = (uint64_t)batch * tq;
  if (rows == 0 || heads == 0) return CATENA_OK;
  if (head_dim == 0 || head_dim % 2 != 0)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "rope needs an even head_dim");
  if (!qkv || !inv_freq || !lens || !q || !k_cache || !v_cache)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  const uint64_t threads = rows * heads * (head_dim / 2);
  if (rows > 0xFFFFFFFFull || ceil_div(threads, 256) > 0x7FFFFFFFull)
    return fail(CATENA_ERR_UNSUPPORTED, "rope shape too large");
  uint32_t R = (uint32_t)rows;
  void* args[] = {&qkv, &inv_freq, &lens, &q, &k_cache, &v_cache, &R, &tq, &heads, &head_dim,
                  &max_len};
  return launch(KernelId::RopeQkvStore, dim3((unsigned)ceil_div(threads, 256)), dim3(256), 0, args);
}

int catena_mi355x_silu_mul_bf16(const float* gu, uint16_t* out, uint64_t rows, uint32_t ffn,
                                uint32_t group) {
  int st = ensure_init();
  if (st) return st;
  if (rows == 0 || ffn == 0) return CATENA_OK;
  if (!gu || !out) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (ffn % 4 != 0 || !aligned16(gu) || (reinterpret_cast<uintptr_t>(out) & 7u))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "silu_mul needs F %% 4 == 0 and aligned rows");
  if (group != 0 && (group % 4 != 0 || ffn % group != 0))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "silu_mul group must divide F and be a multiple of 4");
  if (rows > 65535) return fail(CATENA_ERR_UNSUPPORTED, "silu_mul of more than 65535 rows");
  void* args[] = {&gu, &out, &ffn, &group};
  return launch(KernelId::SiluMulBf16, dim3((unsigned)ceil_div(ffn, 1024), (unsigned)rows),
                dim3(256), 0, args);
}

int catena_mi355x_argmax_f32(const float* x, uint32_t* idx, uint64_t rows, uint64_t n) {
  int st = ensure_init();
  if (st) return st;
  if (rows == 0) return CATENA_OK;
  if (!idx || (n > 0 && !x)) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (rows > 0x7FFFFFFFull || n >= 0x7FFFFFFFull)
    return fail(CATENA_ERR_UNSUPPORTED, "argmax shape too large");
  if (rows > 65535) return fail(CATENA_ERR_UNSUPPORTED, "argmax of more than 65535 rows");
  // Chunks of 4096 elements per workgroup (fewer, longer ones when the
  // per-row partials would not fit the library's scratch).
  const Device& d = device();
  const uint64_t max_parts = Device::kRowPartialBytes / 12;
  uint64_t chunk = 4096;
  if (rows > Device::kTicketsRows) {
    chunk = n > 0 ? n : 1;  // one workgroup per row: no ticket needed
  } else {
    while (rows * ceil_div(n, chunk) > max_parts) chunk *= 2;
  }
  const uint64_t chunks = n > 0 ? ceil_div(n, chunk) : 1;
  uint32_t n32 = (uint32_t)n, chunk32 = (uint32_t)chunk;
  uint32_t* tickets = d.row_tickets();
  uint32_t* partials = static_cast<uint32_t*>(d.row_partials());
  void* args[] = {&x, &idx, &n32, &chunk32, &tickets, &partials};
  return launch(KernelId::ArgmaxRowsF32, dim3((unsigned)chunks, (unsigned)rows), dim3(256), 0, args);
}

// ---------------------------------------------------------------- programs

void program_nn_rmsnorm(catena_mem_t x, catena_mem_t* out) {
  const uint64_t n = x.len / 4;  // mem.cast.f32
  catena_mem_t y{nullptr, 0};
  if (catena_mem_alloc(n * 4, &y) != CATENA_OK) trap_gpu("output allocation");
  if (n > 0) {
    if (catena_mi355x_rmsnorm_f32(static_cast<const float*>(x.data), static_cast<float*>(y.data), 1,
                                  n) != CATENA_OK)
      trap_gpu("nn.rmsnorm");
    if (catena_mi355x_synchronize() != CATENA_OK) trap_gpu("synchronize");
  }
  *out = y;
}

void program_tensor_argmax_f32(catena_mem_t x, uint64_t* out) {
  const uint64_t n = x.len / 4;
  if (n == 0) trap_assert("u64.assert-nz: argmax of an empty buffer");
  catena_mem_t idx{nullptr, 0};
  if (catena_mem_alloc(4, &idx) != CATENA_OK) trap_gpu("output allocation");
  if (catena_mi355x_argmax_f32(static_cast<const float*>(x.data), static_cast<uint32_t*>(idx.data), 1,
                               n) != CATENA_OK)
    trap_gpu("tensor.argmax-f32");
  uint32_t host = 0;
  if (catena_mem_read(idx, 0, &host, 4) != CATENA_OK) trap_gpu("download");
  catena_mem_free(&idx);
  *out = host;
}

}  // extern "C"
