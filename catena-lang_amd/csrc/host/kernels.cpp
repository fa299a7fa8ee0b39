// Kernel ABI: shape checks, kernel selection and launches.
#include <cstdint>
#include <cstdlib>
#include <cstring>

#include "internal.h"

using namespace catena;

namespace {
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// 256 x 128 tiles instead of 256 x 256: measured on the box, a round of
// 256 x 128 tiles (one per CU) takes ~0.6 of a round of 256 x 256 tiles at the
// same K, so the narrow tiles win when the wide ones leave CUs idle (W_o and
// W_down of the C5 prefill: 128 wide tiles for 256 CUs, 52.6 -> 37.6 us and
// 124 -> 93 us) and lose on full rounds (4096^3: 115 -> 138 us).
bool prefer_n128(uint64_t rows, uint64_t cols, int cu_count) {
  const uint64_t cus = cu_count > 0 ? (uint64_t)cu_count : 256;
  const uint64_t wide = (rows / 256) * (cols / 256);
  const uint64_t narrow = (rows / 256) * (cols / 128);
  const double r_wide = (double)ceil_div(wide, cus), r_narrow = (double)ceil_div(narrow, cus);
  return 0.62 * r_narrow < r_wide;
}

// Column blocks x k groups the decode kernel spreads a weight over: the
// MI355X's 256 CUs, one 4-wave workgroup per CU.  A constant, not the
// device's CU count: the k grouping fixes which partial sums are added
// together, so it must depend on the shape alone for the bits to be the same
// on every device (a partitioned MI355X shows fewer CUs).
constexpr uint64_t kDecodeSpread = 256;

// k per wave for the decode kernel, in whole 32-k MFMA steps, from (N, K)
// only.  Streaming path (K % 32 == 0, one 4-wave workgroup per CU for its
// 144 KiB LDS ring; each wave keeps 36 KiB in flight): the fewest k groups
// that still give each of the 256 CUs a workgroup, so one round of
// workgroups streams the weight and few partials are added, but no fewer
// than 8 steps per wave, or 2 when the weight is at most 16 MiB: such a
// kernel is bound by latency, not by HBM, and more workgroups shorten each
// stream (measured: 8 x 2048 x 2048 takes 7.5 us at 2 steps per wave against
// 9.4 us at 8; the C3 shapes and the larger decoder projections are fastest
// at the 8-step floor or within 0.5 us of it).  Register path (K % 32 != 0):
// ~1500 waves.
uint32_t decode_kw(uint64_t n_cols, uint64_t k, bool regs_path) {
  const uint64_t blocks = ceil_div(n_cols, 128);
  uint64_t kw;
  if (!regs_path) {
    // at least 8 steps of 32 k per wave: shorter chunks pay the ring's fill
    // and the partials' reduction more often than they gain in spread
    const uint64_t groups = blocks >= kDecodeSpread ? 1 : kDecodeSpread / blocks;
    kw = ceil_div(k, 4 * groups);
    kw = ceil_div(kw, 32) * 32;
    const uint64_t min_kw = n_cols * k * 2 <= (16ull << 20) ? 64 : 256;
    if (kw < min_kw) kw = min_kw;
  } else {
    kw = ceil_div(k * blocks, 1536);
    kw = ceil_div(kw, 32) * 32;
    if (kw < 64) kw = 64;
  }
  if (kw > k) kw = ceil_div(k, 32) * 32;
  return (uint32_t)kw;
}
}  // namespace

namespace catena {

uint64_t decode_partials_bytes(uint64_t n, uint64_t m, uint64_t k, uint32_t* k_groups) {
  const uint32_t kw = decode_kw(m, k, k % 32 != 0);
  const uint64_t S = ceil_div(ceil_div(k, kw), 4);
  if (k_groups) *k_groups = S > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)S;
  return S > 1 ? S * n * m * sizeof(float) : 0;
}

int gemm_bf16_decode(const uint16_t* a, const uint16_t* b, void* c, uint64_t n, uint64_t m,
                     uint64_t k, DecodeEpilogue epi, const DecodeEpiArgs& ep, void* scratch,
                     uint64_t scratch_bytes, bool whole_k) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0 || m == 0) return CATENA_OK;
  if (n > 16 || k == 0 || m % 8 != 0 || k % 8 != 0 || !aligned16(a) || !aligned16(b) ||
      !aligned16(c))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "decode GEMM shape or alignment");
  Device& d = device();
  const uint32_t M = (uint32_t)n;
  // streaming ring (4 waves x 4 stages x 9 KiB) when K % 32 == 0, else the
  // register path with the reduction buffers only (4 x 8 KiB wave sums + the
  // 16 x 132 f32 tile)
  const bool regs_path = k % 32 != 0;
  if (ep.x_sums && (regs_path || !ep.x_rows_out || !aligned16(ep.x_sums) || ep.x_sums_blocks == 0 ||
                    ep.x_sums_cols == 0 || ep.x_sums_cols >= 0x7FFFFFFFull ||
                    (uint64_t)n * ep.x_sums_blocks * 16 >= (1ull << 31)))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "decode GEMM token composition operands");
  const uint32_t kw =
      whole_k && !regs_path ? (uint32_t)(ceil_div(ceil_div(k, 4), 32) * 32) : decode_kw(m, k, regs_path);
  const uint64_t chunks = ceil_div(k, kw);
  const uint64_t S = ceil_div(chunks, 4);
  const uint64_t gx = ceil_div(m, 128);
  if (S > 65535 || gx > Device::kTicketsGemm)
    return fail(CATENA_ERR_UNSUPPORTED, "decode GEMM grid too large");
  KernelId id = KernelId::GemmBf16DecodeF32;
  DecodeEpiArgs e = ep;
  switch (epi) {
    case DecodeEpilogue::StoreF32: break;
    case DecodeEpilogue::StoreBf16: id = KernelId::GemmBf16DecodeBf16; break;
    case DecodeEpilogue::Rope:
      if (e.heads == 0 || m != 3ull * e.heads * 128 || !e.q_out || !e.k_cache || !e.v_cache ||
          !e.lens || !e.inv_freq)
        return fail(CATENA_ERR_INVALID_ARGUMENT, "rope epilogue operands");
      id = KernelId::GemmBf16DecodeRope;
      break;
    case DecodeEpilogue::Silu:
      if (m % 128 != 0 || !e.act) return fail(CATENA_ERR_INVALID_ARGUMENT, "silu epilogue operands");
      id = KernelId::GemmBf16DecodeSilu;
      break;
    case DecodeEpilogue::Partials:
      id = KernelId::GemmBf16DecodeParts;
      break;
    case DecodeEpilogue::Argmax:
      if ((!e.idx && !e.arg_defer) || m >= 0x7FFFFFFFull)
        return fail(CATENA_ERR_INVALID_ARGUMENT, "argmax epilogue operands");
      if (n * gx * 16 > Device::kRowPartialBytes)
        return fail(CATENA_ERR_UNSUPPORTED, "argmax epilogue over %llu column blocks",
                    (unsigned long long)gx);
      e.arg_ticket = d.misc_tickets();
      if (!e.arg_partials) e.arg_partials = static_cast<uint32_t*>(d.row_partials());
      else if (!aligned16(e.arg_partials))
        return fail(CATENA_ERR_INVALID_ARGUMENT, "argmax summaries must be 16-byte aligned");
      id = KernelId::GemmBf16DecodeArgmax;
      break;
  }
  float* P = nullptr;
  std::lock_guard<std::mutex> ws_guard(d.ws_mu);  // the workspace block stays ours until launched
  if (S > 1) {
    // the partials are addressed through one buffer descriptor with 32-bit
    // byte offsets
    const uint64_t pbytes = S * M * m * sizeof(float);
    if (pbytes >= (1ull << 31))
      return fail(CATENA_ERR_UNSUPPORTED, "decode GEMM partials exceed 2 GiB (%llu k groups)",
                  (unsigned long long)S);
    if (scratch) {
      // caller-provided scratch (the allocation-free entry point)
      if (pbytes > scratch_bytes)
        return fail(CATENA_ERR_UNSUPPORTED,
                    "decode GEMM partials need %llu B of scratch, more than the %llu B available",
                    (unsigned long long)pbytes, (unsigned long long)scratch_bytes);
      P = static_cast<float*>(scratch);
    } else {
      void* ws = nullptr;
      st = workspace(pbytes, &ws);
      if (st) return st;
      P = static_cast<float*>(ws);
    }
  }
  const uint16_t* X = a;
  const uint16_t* W = b;
  void* Y = c;
  uint64_t N = m, K = k;
  uint32_t* tickets = d.gemm_tickets();
  uint32_t stream_lds = regs_path ? 0u : 1u;
  const size_t lds = stream_lds ? 4 * 4 * 9216 : 4 * 8 * 64 * 16 + 16 * 132 * 4;
  void* args[] = {&X, &W, &Y, &P, &tickets, (void*)&M, &N, &K, (void*)&kw, &stream_lds, &e};
  if (lds > d.max_lds) return fail(CATENA_ERR_UNSUPPORTED, "decode GEMM needs %zu B of LDS", lds);
  if (S > 1 && (epi == DecodeEpilogue::StoreF32 || epi == DecodeEpilogue::StoreBf16)) {
    // plain output: the partials kernel (W streamed non-temporally, as the
    // plain-output kernels do), then the reduction as a launch of its own
    // (the same adds in the same order, ordered by the launch boundary
    // instead of a completion ticket)
    st = launch(KernelId::GemmBf16DecodePartsNt, dim3((unsigned)gx, (unsigned)S), dim3(256), lds, args);
    if (st) return st;
    uint64_t part_elems = (uint64_t)M * m, n4 = part_elems / 4;
    uint32_t S32 = (uint32_t)S, bf16 = epi == DecodeEpilogue::StoreBf16 ? 1u : 0u;
    void* rargs[] = {&P, &part_elems, &S32, &Y, &n4, &bf16};
    return launch(KernelId::DecodeReduce, dim3((unsigned)ceil_div(n4, 256)), dim3(256), 0, rargs);
  }
  return launch(id, dim3((unsigned)gx, (unsigned)S), dim3(256), lds, args);
}

int argmax_compose(const uint32_t* sums, uint32_t n, uint32_t blocks, uint64_t cols, uint32_t* idx) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0) return CATENA_OK;
  if (!sums || !idx || n > 16 || blocks == 0 || cols == 0 || cols >= 0x7FFFFFFFull ||
      (uint64_t)n * blocks * 16 >= (1ull << 31))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "argmax composition operands");
  void* args[] = {&sums, &n, &blocks, &cols, &idx};
  return launch(KernelId::ArgmaxCompose, dim3(1), dim3(256), 0, args);
}

int gemm_bf16_decode_parts(const uint16_t* a, const uint16_t* b, float* parts, uint64_t parts_bytes,
                           uint64_t n, uint64_t m, uint64_t k, uint32_t* k_groups,
                           const DecodeEpiArgs& gather) {
  if (!parts || !k_groups) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  uint32_t S = 0;
  decode_partials_bytes(n, m, k, &S);
  *k_groups = S > 0 ? S : 1;
  if ((uint64_t)*k_groups * n * m * sizeof(float) > parts_bytes)
    return fail(CATENA_ERR_UNSUPPORTED, "decode GEMM partials need %llu B",
                (unsigned long long)((uint64_t)*k_groups * n * m * sizeof(float)));
  // S > 1: the partials go to P = parts; S = 1: the product goes to Y = parts
  // (gather: only its X-row fields are read)
  DecodeEpiArgs e;
  e.x_rows = gather.x_rows;
  e.x_rows_limit = gather.x_rows_limit;
  e.x_sums = gather.x_sums;
  e.x_sums_blocks = gather.x_sums_blocks;
  e.x_sums_cols = gather.x_sums_cols;
  e.x_rows_out = gather.x_rows_out;
  return gemm_bf16_decode(a, b, parts, n, m, k, DecodeEpilogue::Partials, e, parts, parts_bytes);
}

bool attn_few_fits(uint32_t batch, uint32_t tq, uint32_t heads, uint32_t max_len) {
  const uint64_t nq = (uint64_t)batch * tq * heads;
  return nq > 0 && nq <= kAttnFewMaxQueries && tq < 8 && max_len >= 64 &&
         attn_few_lds_bytes(max_len) <= device().max_lds;
}

int attn_few_launch(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint32_t* lens,
                    void* o, uint32_t batch, uint32_t tq, uint32_t heads, uint32_t max_len,
                    float scale, bool out_f32, const FewQkvArgs& qkv) {
  const uint64_t nq = (uint64_t)batch * tq * heads;
  if (!attn_few_fits(batch, tq, heads, max_len)) return -1;
  if (qkv.parts && (tq != 1 || qkv.n_parts == 0 || !qkv.rope_tab || !qkv.q_out || !qkv.k_cache ||
                    !qkv.v_cache || qkv.part_stride < (uint64_t)batch * 3 * heads * 128))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "attention q/k/v partials operands");
  FewQkvArgs a = qkv;
  void* args[] = {&q, &k, &v, &lens, &o, &heads, &max_len, &tq, &scale, &a};
  // up to 128 pairs: two workgroups per pair (each makes all the scores and
  // adds one half of the output columns), so that 2 x pairs CUs stream K
  // and V instead of one per pair
  if (nq <= kAttnFewSplitMaxQueries)
    return launch(out_f32 ? KernelId::AttnFewSplitD128F32 : KernelId::AttnFewSplitD128Bf16,
                  dim3((unsigned)(2 * nq)), dim3(448), attn_few_split_lds_bytes(max_len), args);
  return launch(out_f32 ? KernelId::AttnFewD128F32 : KernelId::AttnFewD128Bf16, dim3((unsigned)nq),
                dim3(512), attn_few_lds_bytes(max_len), args);
}

bool gemm_bf16_silu_fits(uint64_t n, uint64_t m, uint64_t k, const void* a, const void* b,
                         const void* act) {
  return n % 256 == 0 && m % 128 == 0 && k % 128 == 0 && k > 0 && k <= (1ull << 22) &&
         m <= (1ull << 24) && aligned16(a) && aligned16(b) && aligned16(act) &&
         (n / 256) * (m / 128) <= 0x7FFFFFFFull;
}

bool gemm_bf16_rope_fits(uint64_t rows, uint64_t k, uint32_t tq, uint32_t heads, const void* a,
                         const void* w, const void* q_out, const void* kc, const void* vc,
                         const void* tab) {
  const uint64_t m = 3ull * heads * 128;
  return tq > 0 && heads > 0 && rows % 256 == 0 && rows % tq == 0 && k % 128 == 0 && k > 0 &&
         k <= (1ull << 22) && m <= (1ull << 24) && aligned16(a) && aligned16(w) && aligned16(q_out) &&
         aligned16(kc) && aligned16(vc) && aligned16(tab) && (rows / 256) * (m / 128) <= 0x7FFFFFFFull;
}

bool gemm_bf16_ksplit_fits(uint64_t n, uint64_t m, uint64_t k, uint32_t splits, const void* a,
                           const void* b, const void* parts) {
  return splits > 0 && splits <= 64 && n % 256 == 0 && m % 256 == 0 && k > 0 &&
         k % (128ull * splits) == 0 && k <= (1ull << 22) && m <= (1ull << 24) && aligned16(a) &&
         aligned16(b) && aligned16(parts) && (n / 256) * (m / 256) <= 0x7FFFFFFFull;
}

int gemm_bf16_f32_ksplit(const uint16_t* a, const uint16_t* b, float* parts, uint64_t n, uint64_t m,
                         uint64_t k, uint32_t splits) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0 || m == 0) return CATENA_OK;
  if (!a || !b || !parts) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (!gemm_bf16_ksplit_fits(n, m, k, splits, a, b, parts))
    return fail(CATENA_ERR_UNSUPPORTED, "k-split GEMM: shape or alignment not taken");
  const size_t lds = 4ull * (256 + 256) * 32 * sizeof(uint16_t);
  if (lds > device().max_lds) return fail(CATENA_ERR_UNSUPPORTED, "device LDS %zu < %zu", device().max_lds, lds);
  uint64_t k_len = k / splits;
  void* args[] = {&a, &b, &parts, &n, &m, &k, &k_len};
  return launch(KernelId::GemmBf16K32F32Parts, dim3((unsigned)((n / 256) * (m / 256)), splits), dim3(512), lds,
                args);
}

int gemm_bf16_rope_qkv(const uint16_t* a, const uint16_t* w, const float* tab, const uint32_t* lens,
                       uint16_t* q_out, uint16_t* kc, uint16_t* vc, uint64_t rows, uint64_t k,
                       uint32_t tq, uint32_t heads, uint32_t max_len) {
  int st = ensure_init();
  if (st) return st;
  if (rows == 0) return CATENA_OK;
  if (!a || !w || !tab || !lens || !q_out || !kc || !vc)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (!gemm_bf16_rope_fits(rows, k, tq, heads, a, w, q_out, kc, vc, tab))
    return fail(CATENA_ERR_UNSUPPORTED, "fused q / k / v projection: shape or alignment not taken");
  // the stages (4 x (256 + 128) x 32 bf16) hold the epilogue's staging,
  // 8 waves x 64 rows x 128 bytes
  const size_t lds = 4ull * (256 + 128) * 32 * sizeof(uint16_t);
  if (lds > device().max_lds) return fail(CATENA_ERR_UNSUPPORTED, "device LDS %zu < %zu", device().max_lds, lds);
  uint64_t n = rows, m = 3ull * heads * 128;
  const uint64_t grid = (n / 256) * (m / 128);
  void* args[] = {&a, &w, &n, &m, &k, &tab, &lens, &q_out, &kc, &vc, &tq, &heads, &max_len};
  return launch(KernelId::GemmBf16K32N128Rope, dim3((unsigned)grid), dim3(512), lds, args);
}

}  // namespace catena

extern "C" {

int catena_mi355x_gemm_f32_exact(const float* a, const float* b, float* c, uint64_t n, uint64_t m,
                                 uint64_t k) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0 || m == 0) return CATENA_OK;
  if (!c || (k > 0 && (!a || !b))) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  void* args[] = {&a, &b, &c, &n, &m, &k};
  // 64x64 tiles (16 cells per thread) unless they would leave CUs idle; then
  // 16x16 tiles with one cell per thread: A by DPP row broadcast and B through
  // LDS when k % 16 == 0, B's rows are 16-byte aligned and the buffer offsets
  // fit 31 bits, else A and B both through LDS.  Every cell is the same
  // k-ascending chain in all three, so the choice never changes the bits.
  const uint64_t gx = ceil_div(m, 64), gy = ceil_div(n, 64);
  if (gx * gy < kDecodeSpread) {
    const uint64_t sx = ceil_div(m, 16), sy = ceil_div(n, 16);
    if (k > 0 && k % 16 == 0 && m % 4 == 0 && aligned16(b) && reinterpret_cast<uintptr_t>(a) % 4 == 0 &&
        (n + 16) * k * 4 < (1ull << 31) && (k + 256) * m * 4 < (1ull << 31) && sy <= 65535)
      return launch(KernelId::GemmF32ExactQ16, dim3((unsigned)sx, (unsigned)sy), dim3(256), 256 * 16 * 4, args);
    return launch(KernelId::GemmF32ExactT16, dim3((unsigned)sx, (unsigned)sy), dim3(256), 0, args);
  }
  if (gx > 0x7FFFFFFFu || gy > 65535u) return fail(CATENA_ERR_UNSUPPORTED, "matrix too large");
  return launch(KernelId::GemmF32Exact, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, args);
}

int catena_mi355x_gemm_bf16(const uint16_t* a, const uint16_t* b, void* c, uint64_t n, uint64_t m,
                            uint64_t k, int out_f32) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0 || m == 0) return CATENA_OK;
  if (!c || (k > 0 && (!a || !b))) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  Device& d = device();

  // decode shape: <= 16 rows of activations against a K x N weight
  if (n <= 16 && k > 0 && m % 8 == 0 && k % 8 == 0 && aligned16(a) && aligned16(b) &&
      aligned16(c))
    return gemm_bf16_decode(a, b, c, n, m, k,
                            out_f32 ? DecodeEpilogue::StoreF32 : DecodeEpilogue::StoreBf16,
                            DecodeEpiArgs{}, nullptr, 0);

  const bool ptr_ok = aligned16(a) && aligned16(b) && aligned16(c);
  const bool tile_ok = n % 256 == 0 && m % 256 == 0 && k % 64 == 0 && k > 0 && ptr_ok;
  // the 32-k stage kernels need K % 128 == 0 (whole groups of 4 stages);
  // they address A's 256-row tile and B's 32-row slab with
  // 32-bit buffer offsets
  const bool k32_ok = k % 128 == 0 && k > 0 && k <= (1ull << 22) && m <= (1ull << 24);
  const bool n128_ok = n % 256 == 0 && m % 128 == 0 && k32_ok && ptr_ok;
  const uint64_t tiles = ceil_div(n, 256) * ceil_div(m, 256);
  if (ceil_div(n, 256) * ceil_div(m, 128) > 0x7FFFFFFFu)
    return fail(CATENA_ERR_UNSUPPORTED, "matrix too large");
  void* args[] = {&a, &b, &c, &n, &m, &k};
  // Aligned shapes: direct-to-LDS kernels (8 waves), all with the same
  // per-accumulator k32 order, so the choice between them never changes the
  // bits: the four-stage 32-k kernel on 256 x 256 tiles, or on 256 x 128
  // tiles when N % 256 == 128 or when that takes fewer rounds of the chip;
  // the two-stage 64-k kernel when K % 128 != 0.
  if (tile_ok || n128_ok) {
    KernelId id;
    size_t lds;
    uint64_t grid;
    if (k32_ok && (!tile_ok || prefer_n128(n, m, d.cu_count))) {
      id = out_f32 ? KernelId::GemmBf16K32N128F32 : KernelId::GemmBf16K32N128Bf16;
      lds = 4ull * (256 + 128) * 32 * sizeof(uint16_t);  // 98304 B
      grid = (n / 256) * (m / 128);
    } else if (k32_ok) {
      id = out_f32 ? KernelId::GemmBf16K32F32 : KernelId::GemmBf16K32Bf16;
      lds = 4ull * (256 + 256) * 32 * sizeof(uint16_t);  // 131072 B
      grid = tiles;
    } else {
      id = out_f32 ? KernelId::GemmBf16LdsF32 : KernelId::GemmBf16LdsBf16;
      lds = 2ull * (256 * 64 + 64 * 256) * sizeof(uint16_t);  // 131072 B
      grid = tiles;
    }
    if (lds > d.max_lds) return fail(CATENA_ERR_UNSUPPORTED, "device LDS %zu < %zu", d.max_lds, lds);
    return launch(id, dim3((unsigned)grid), dim3(512), lds, args);
  }
  const size_t lds = 2ull * 2 * 256 * 72 * sizeof(uint16_t);  // 147456 B
  if (lds > d.max_lds) return fail(CATENA_ERR_UNSUPPORTED, "device LDS %zu < %zu", d.max_lds, lds);
  return launch(out_f32 ? KernelId::GemmBf16EdgeF32 : KernelId::GemmBf16EdgeBf16,
                dim3((unsigned)tiles), dim3(256), lds, args);
}

int catena_mi355x_gemm_bf16_silu(const uint16_t* a, const uint16_t* b, uint16_t* act, uint64_t n,
                                 uint64_t m, uint64_t k) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0 || m == 0) return CATENA_OK;
  if (!act || (k > 0 && (!a || !b))) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (!gemm_bf16_silu_fits(n, m, k, a, b, act))
    return fail(CATENA_ERR_UNSUPPORTED,
                "SwiGLU GEMM needs n %% 256 == 0, m %% 128 == 0, k %% 128 == 0 (k <= 2^22, m <= 2^24) "
                "and 16-byte aligned pointers");
  Device& d = device();
  // the tile width the plain GEMM would take for this shape (same bits)
  const bool narrow = m % 256 != 0 || prefer_n128(n, m, d.cu_count);
  const size_t stages = narrow ? 4ull * (256 + 128) * 32 * sizeof(uint16_t)   // 98304 B
                               : 4ull * (256 + 256) * 32 * sizeof(uint16_t);  // 131072 B
  const size_t slots = 4ull * (narrow ? 64 : 128) * 68 * sizeof(float);        // up-column hand-over
  const size_t lds = stages > slots ? stages : slots;
  if (lds > d.max_lds) return fail(CATENA_ERR_UNSUPPORTED, "device LDS %zu < %zu", d.max_lds, lds);
  const uint64_t grid = narrow ? (n / 256) * (m / 128) : (n / 256) * (m / 256);
  void* args[] = {&a, &b, &act, &n, &m, &k};
  return launch(narrow ? KernelId::GemmBf16K32N128Silu : KernelId::GemmBf16K32Silu, dim3((unsigned)grid),
                dim3(512), lds, args);
}

int catena_mi355x_gemm_bf16_rope_qkv(const uint16_t* a, const uint16_t* w, const float* rope_tab,
                                     const uint32_t* lens, uint16_t* q, uint16_t* k_cache,
                                     uint16_t* v_cache, uint32_t batch, uint32_t tq, uint32_t heads,
                                     uint32_t max_len, uint64_t k) {
  int st = ensure_init();
  if (st) return st;
  const uint64_t rows = (uint64_t)batch * tq;
  if (rows == 0 || heads == 0) return CATENA_OK;
  if (!a || !w || !rope_tab || !lens || !q || !k_cache || !v_cache)
    return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (!gemm_bf16_rope_fits(rows, k, tq, heads, a, w, q, k_cache, v_cache, rope_tab))
    return fail(CATENA_ERR_UNSUPPORTED,
                "fused q / k / v projection needs batch * tq %% 256 == 0, k %% 128 == 0 (k <= 2^22) "
                "and 16-byte aligned pointers");
  return gemm_bf16_rope_qkv(a, w, rope_tab, lens, q, k_cache, v_cache, rows, k, tq, heads, max_len);
}

int catena_mi355x_gemm_bf16_ksplit_f32(const uint16_t* a, const uint16_t* b, float* parts,
                                       uint64_t n, uint64_t m, uint64_t k, uint32_t splits) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0 || m == 0) return CATENA_OK;
  if (!a || !b || !parts) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (!gemm_bf16_ksplit_fits(n, m, k, splits, a, b, parts))
    return fail(CATENA_ERR_UNSUPPORTED,
                "k-split GEMM needs 1 <= splits <= 64, n %% 256 == 0, m %% 256 == 0, "
                "k %% (128 splits) == 0 (k <= 2^22) and 16-byte aligned pointers");
  return gemm_bf16_f32_ksplit(a, b, parts, n, m, k, splits);
}

int catena_mi355x_gemm_bf16_argmax(const uint16_t* a, const uint16_t* b, float* c, uint32_t* idx,
                                   uint64_t n, uint64_t m, uint64_t k) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0 || m == 0) return CATENA_OK;
  if (!a || !b || !c || !idx) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  DecodeEpiArgs e;
  e.idx = idx;
  return gemm_bf16_decode(a, b, c, n, m, k, DecodeEpilogue::Argmax, e);
}

int catena_mi355x_attn_decode_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                   const uint32_t* lens, float* o, uint32_t batch, uint32_t heads,
                                   uint32_t max_len, uint32_t head_dim, float scale) {
  int st = ensure_init();
  if (st) return st;
  if (head_dim != 128)
    return fail(CATENA_ERR_UNSUPPORTED, "attention head_dim %u unsupported (only 128)", head_dim);
  const uint64_t bh = (uint64_t)batch * heads;
  if (bh == 0) return CATENA_OK;
  if (!q || !lens || !o || (max_len > 0 && (!k || !v)))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (!aligned16(k) || !aligned16(v))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "K/V caches must be 16-byte aligned");
  if (bh > 0x7FFFFFFFu) return fail(CATENA_ERR_UNSUPPORTED, "too many heads");
  Device& d = device();
  const size_t lds = attn_lds_bytes(max_len);
  if (lds > d.max_lds)
    return fail(CATENA_ERR_UNSUPPORTED, "max_len %u needs %zu B of LDS (device has %zu)", max_len,
                lds, d.max_lds);
  // few (batch, head) pairs: the eight-wave kernel spreads each over a CU
  st = attn_few_launch(q, k, v, lens, o, batch, 1, heads, max_len, scale, true);
  if (st >= 0) return st;
  void* args[] = {&q, &k, &v, &lens, &o, &heads, &max_len, &scale};
  return launch(KernelId::AttnDecodeD128, dim3((unsigned)bh), dim3(256), lds, args);
}

int catena_mi355x_softmax_f32(const float* x, float* y, uint64_t rows, uint64_t n) {
  int st = ensure_init();
  if (st) return st;
  if (rows == 0 || n == 0) return CATENA_OK;
  if (!x || !y) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (n >= 0x7FFFFFFFull) return fail(CATENA_ERR_UNSUPPORTED, "softmax length too large");
  if (rows > 0x7FFFFFFFull) return fail(CATENA_ERR_UNSUPPORTED, "too many rows");
  void* args[] = {&x, &y, &n};
  return launch(KernelId::SoftmaxRows, dim3((unsigned)rows), dim3(256), 0, args);
}

int catena_mi355x_exp_approx_f32(const float* x, float* y, uint64_t n) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0) return CATENA_OK;
  if (!x || !y) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  const uint64_t g = ceil_div(n, 256);
  if (g > 0x7FFFFFFFull) return fail(CATENA_ERR_UNSUPPORTED, "too many elements");
  void* args[] = {&x, &y, &n};
  return launch(KernelId::ExpApprox, dim3((unsigned)g), dim3(256), 0, args);
}

int catena_mi355x_map_f32(uint32_t op, const float* x, float* y, uint64_t n) {
  if (op > CATENA_MAP_SIN_APPROX_FULL) return fail(CATENA_ERR_INVALID_ARGUMENT, "unknown map op %u", op);
  int st = ensure_init();
  if (st) return st;
  if (n == 0) return CATENA_OK;
  if (!x || !y) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  const uint64_t g = ceil_div(n, 256);
  if (g > 0x7FFFFFFFull) return fail(CATENA_ERR_UNSUPPORTED, "too many elements");
  void* args[] = {&x, &y, &n, &op};
  return launch(KernelId::MapF32, dim3((unsigned)g), dim3(256), 0, args);
}

int catena_mi355x_fill_normal_bf16(uint16_t* out, uint64_t n, uint64_t seed, uint64_t stream,
                                   float scale) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0) return CATENA_OK;
  if (!out) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  const uint64_t g = ceil_div(n, 256);
  if (g > 0x7FFFFFFFull) return fail(CATENA_ERR_UNSUPPORTED, "too many elements");
  void* args[] = {&out, &n, &seed, &stream, &scale};
  return launch(KernelId::FillNormalBf16, dim3((unsigned)g), dim3(256), 0, args);
}

int catena_mi355x_fill_uniform_f32(float* out, uint64_t n, uint64_t seed, uint64_t stream) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0) return CATENA_OK;
  if (!out) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  const uint64_t g = ceil_div(n, 256);
  if (g > 0x7FFFFFFFull) return fail(CATENA_ERR_UNSUPPORTED, "too many elements");
  void* args[] = {&out, &n, &seed, &stream};
  return launch(KernelId::FillUniformF32, dim3((unsigned)g), dim3(256), 0, args);
}

int catena_mi355x_gemm_bf16_decode_plan(uint64_t n, uint64_t m, uint64_t k, uint32_t* k_groups,
                                        uint64_t* partials_bytes) {
  if (!k_groups || !partials_bytes) return fail(CATENA_ERR_INVALID_ARGUMENT, "null output");
  *k_groups = 0;
  *partials_bytes = 0;
  if (n == 0 || n > 16 || m == 0 || k == 0 || m % 8 != 0 || k % 8 != 0)
    return fail(CATENA_ERR_INVALID_ARGUMENT,
                "not a decode-GEMM shape (1 <= n <= 16, m %% 8 == 0, k %% 8 == 0, k > 0)");
  *partials_bytes = decode_partials_bytes(n, m, k, k_groups);
  return CATENA_OK;
}

int catena_mi355x_copy_bytes(void* dst, const void* src, uint64_t n) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0) return CATENA_OK;
  if (!dst || !src) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  if (n % 16 != 0 || !aligned16(dst) || !aligned16(src))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "copy needs 16-byte aligned pointers and size");
  uint64_t n16 = n / 16;
  const uint64_t g = ceil_div(n16, 256) < 8192 ? ceil_div(n16, 256) : 8192;
  void* args[] = {&dst, &src, &n16};
  return launch(KernelId::Copy16, dim3((unsigned)g), dim3(256), 0, args);
}

}  // extern "C"
