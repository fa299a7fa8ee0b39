// Kernel ABI: shape checks, variant selection and launches.
#include <cstdint>
#include <cstdlib>
#include <cstring>

#include "internal.h"

using namespace catena;

namespace {
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// Aligned-shape bf16 GEMM kernels.  All compute the same 256x256 tiles with
// the same per-accumulator k32 order (bitwise identical outputs); they differ
// in scheduling only.  CATENA_GEMM_VARIANT selects one for comparison.
struct GemmVariant {
  KernelId bf16, f32;
  uint64_t min_k;  // K must be a multiple of 64 and at least this
};
const GemmVariant kGemmVariants[] = {
    /* 0 two barriers per 64-k slab */
    {KernelId::GemmBf16LdsV0Bf16, KernelId::GemmBf16LdsV0F32, 64},
    /* 1 v0 + MFMA priority */
    {KernelId::GemmBf16LdsV1Bf16, KernelId::GemmBf16LdsV1F32, 64},
    /* 2 one barrier per slab, fragment double-buffering */
    {KernelId::GemmBf16LdsV2Bf16, KernelId::GemmBf16LdsV2F32, 64},
    /* 3 v2 + MFMA priority */
    {KernelId::GemmBf16LdsV3Bf16, KernelId::GemmBf16LdsV3F32, 64},
    /* 4 v2 with LDS reads interleaved 1:2 with MFMAs */
    {KernelId::GemmBf16LdsV4Bf16, KernelId::GemmBf16LdsV4F32, 64},
    /* 5 v4 + MFMA priority */
    {KernelId::GemmBf16LdsV5Bf16, KernelId::GemmBf16LdsV5F32, 64},
    /* 6 four 32-k stages, three slabs in flight (gemm_bf16_deep.hip) */
    {KernelId::GemmBf16DeepBf16, KernelId::GemmBf16DeepF32, 128},
    /* 7 v4 with reads front-loaded 1:1 */
    {KernelId::GemmBf16LdsV7Bf16, KernelId::GemmBf16LdsV7F32, 64},
    /* 8 v6 with reads front-loaded 1:1 */
    {KernelId::GemmBf16DeepFrontBf16, KernelId::GemmBf16DeepFrontF32, 128},
    /* 9 four 32-k stages through buffer loads spread over the MFMAs, LDS-staged
       bf16 epilogue (gemm_bf16_k32.hip) */
    {KernelId::GemmBf16K32Bf16, KernelId::GemmBf16K32F32, 128},
    /* 10 variant 9 on 256 x 128 tiles (8 waves of 64 x 64) */
    {KernelId::GemmBf16K32N128Bf16, KernelId::GemmBf16K32N128F32, 128},
};
constexpr int kGemmVariantCount = sizeof(kGemmVariants) / sizeof(kGemmVariants[0]);
// Default: variant 9 when K % 128 == 0 (and its 32-bit buffer offsets hold),
// else variant 7; variant 9 on 256 x 128 tiles (10) when that takes fewer
// rounds of the chip (see prefer_n128).
constexpr int kGemmDefaultVariant = 9;
constexpr int kGemmFallbackVariant = 7;
constexpr int kGemmN128Variant = 10;

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

// k per wave for the decode kernel, in whole 32-k MFMA steps.
// Streaming path (K % 32 == 0, one 4-wave workgroup per CU for its 144 KiB
// LDS ring; each wave keeps 36 KiB in flight): the fewest k groups that
// still give every CU a workgroup, so one round of workgroups streams the
// weight and few partials are added, but no fewer than 8 steps per wave,
// or 2 when the weight is at most 16 MiB: such a kernel is bound by
// latency, not by HBM, and more workgroups shorten each stream (measured:
// 8 x 2048 x 2048 takes 7.5 us at 2 steps per wave against 9.4 us at 8;
// the C3 shapes and the larger decoder projections are fastest at the
// 8-step floor or within 0.5 us of it).  Register path: ~1500 waves.
// CATENA_DECODE_KW overrides.
uint32_t decode_kw(uint64_t n_cols, uint64_t k, int cu_count, bool regs_path) {
  const char* env = getenv("CATENA_DECODE_KW");
  if (env && *env) {
    long v = strtol(env, nullptr, 10);
    if (v >= 32 && v % 32 == 0) return (uint32_t)v;
  }
  const uint64_t blocks = ceil_div(n_cols, 128);
  uint64_t kw;
  if (!regs_path) {
    // at least 8 steps of 32 k per wave: shorter chunks pay the ring's fill
    // and the partials' reduction more often than they gain in spread
    uint64_t groups = blocks >= (uint64_t)cu_count ? 1 : (uint64_t)cu_count / blocks;
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

int gemm_bf16_decode(const uint16_t* a, const uint16_t* b, void* c, uint64_t n, uint64_t m,
                     uint64_t k, DecodeEpilogue epi, const DecodeEpiArgs& ep) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0 || m == 0) return CATENA_OK;
  if (n > 16 || k == 0 || m % 8 != 0 || k % 8 != 0 || !aligned16(a) || !aligned16(b) ||
      !aligned16(c))
    return fail(CATENA_ERR_INVALID_ARGUMENT, "decode GEMM shape or alignment");
  Device& d = device();
  const uint32_t M = (uint32_t)n;
  const char* dpath = getenv("CATENA_DECODE_PATH");
  const bool regs_path = k % 32 != 0 || (dpath && strcmp(dpath, "regs") == 0);
  const uint32_t kw = decode_kw(m, k, d.cu_count > 0 ? d.cu_count : 256, regs_path);
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
    case DecodeEpilogue::Argmax:
      if (!e.idx || m >= 0x7FFFFFFFull) return fail(CATENA_ERR_INVALID_ARGUMENT, "argmax epilogue operands");
      if (n * gx * 16 > Device::kRowPartialBytes)
        return fail(CATENA_ERR_UNSUPPORTED, "argmax epilogue over %llu column blocks",
                    (unsigned long long)gx);
      e.arg_ticket = d.misc_tickets();
      e.arg_partials = static_cast<uint32_t*>(d.row_partials());
      id = KernelId::GemmBf16DecodeArgmax;
      break;
  }
  float* P = nullptr;
  std::lock_guard<std::mutex> ws_guard(d.ws_mu);  // the workspace block stays ours until launched
  if (S > 1) {
    // the partials are addressed through one buffer descriptor with 32-bit
    // byte offsets
    if (S * M * m * sizeof(float) >= (1ull << 31))
      return fail(CATENA_ERR_UNSUPPORTED, "decode GEMM partials exceed 2 GiB (%llu k groups)",
                  (unsigned long long)S);
    void* ws = nullptr;
    st = workspace(S * M * m * sizeof(float), &ws);
    if (st) return st;
    P = static_cast<float*>(ws);
  }
  const uint16_t* X = a;
  const uint16_t* W = b;
  void* Y = c;
  uint64_t N = m, K = k;
  uint32_t* tickets = d.gemm_tickets();
  // streaming ring (4 waves x 4 stages x 9 KiB) when K % 32 == 0, else the
  // reduction buffers only (3 x 8 KiB partials + the 16 x 132 f32 tile);
  // CATENA_DECODE_PATH=regs selects the register path for comparison
  const char* path = getenv("CATENA_DECODE_PATH");
  uint32_t stream_lds = (k % 32 == 0 && !(path && strcmp(path, "regs") == 0)) ? 1u : 0u;
  const size_t lds = stream_lds ? 4 * 4 * 9216 : 3 * 8 * 64 * 16 + 16 * 132 * 4;
  void* args[] = {&X, &W, &Y, &P, &tickets, (void*)&M, &N, &K, (void*)&kw, &stream_lds, &e};
  if (lds > d.max_lds) return fail(CATENA_ERR_UNSUPPORTED, "decode GEMM needs %zu B of LDS", lds);
  return launch(id, dim3((unsigned)gx, (unsigned)S), dim3(256), lds, args);
}

bool gemm_bf16_silu_fits(uint64_t n, uint64_t m, uint64_t k, const void* a, const void* b,
                         const void* act) {
  return n % 256 == 0 && m % 128 == 0 && k % 128 == 0 && k > 0 && k <= (1ull << 22) &&
         m <= (1ull << 24) && aligned16(a) && aligned16(b) && aligned16(act) &&
         (n / 256) * (m / 128) <= 0x7FFFFFFFull;
}

}  // namespace catena

extern "C" {

int catena_mi355x_gemm_f32_exact(const float* a, const float* b, float* c, uint64_t n, uint64_t m,
                                 uint64_t k) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0 || m == 0) return CATENA_OK;
  if (!c || (k > 0 && (!a || !b))) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  const uint64_t gx = ceil_div(m, 64), gy = ceil_div(n, 64);
  if (gx > 0x7FFFFFFFu || gy > 65535u) return fail(CATENA_ERR_UNSUPPORTED, "matrix too large");
  void* args[] = {&a, &b, &c, &n, &m, &k};
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
                            DecodeEpiArgs{});

  const bool ptr_ok = aligned16(a) && aligned16(b) && aligned16(c);
  const bool tile_ok = n % 256 == 0 && m % 256 == 0 && k % 64 == 0 && k > 0 && ptr_ok;
  // the 32-k stage kernels need K % 128 == 0 (whole groups of 4 stages);
  // variants 9 and 10 address A's 256-row tile and B's 32-row slab with
  // 32-bit buffer offsets
  const bool k32_ok = k % 128 == 0 && k > 0 && k <= (1ull << 22) && m <= (1ull << 24);
  const bool n128_ok = n % 256 == 0 && m % 128 == 0 && k32_ok && ptr_ok;
  const uint64_t tiles = ceil_div(n, 256) * ceil_div(m, 256);
  if (ceil_div(n, 256) * ceil_div(m, 128) > 0x7FFFFFFFu)
    return fail(CATENA_ERR_UNSUPPORTED, "matrix too large");
  void* args[] = {&a, &b, &c, &n, &m, &k};
  // Aligned shapes: direct-to-LDS kernels (8 waves).  The older
  // register-staged tile kernel stays selectable with CATENA_GEMM_TILE=regs
  // for comparison; it computes in the same order per output tile.
  const char* sel = getenv("CATENA_GEMM_TILE");
  const bool use_regs = sel && strcmp(sel, "regs") == 0;
  if ((tile_ok || n128_ok) && !use_regs) {
    int variant = kGemmDefaultVariant;
    const char* v = getenv("CATENA_GEMM_VARIANT");
    const bool forced = v && *v;
    if (forced) {
      const long x = strtol(v, nullptr, 10);
      if (x >= 0 && x < kGemmVariantCount) variant = (int)x;
    }
    if (!tile_ok || (!forced && n128_ok && prefer_n128(n, m, d.cu_count))) variant = kGemmN128Variant;
    if (variant == kGemmN128Variant && !n128_ok) variant = kGemmDefaultVariant;
    if (k < kGemmVariants[variant].min_k || (kGemmVariants[variant].min_k == 128 && !k32_ok))
      variant = kGemmFallbackVariant;
    const GemmVariant& gv = kGemmVariants[variant];
    const bool narrow = variant == kGemmN128Variant;
    // two-stage kernels: 2 x (A 256x64 + B 64x256); four-stage: 4 x (A 256x32 + B 32xBN)
    const size_t lds = narrow ? 4ull * (256 + 128) * 32 * sizeof(uint16_t)   // 98304 B
                              : 2ull * (256 * 64 + 64 * 256) * sizeof(uint16_t);  // 131072 B
    if (lds > d.max_lds) return fail(CATENA_ERR_UNSUPPORTED, "device LDS %zu < %zu", d.max_lds, lds);
    const uint64_t grid = narrow ? (n / 256) * (m / 128) : tiles;
    return launch(out_f32 ? gv.f32 : gv.bf16, dim3((unsigned)grid), dim3(512), lds, args);
  }
  const size_t lds = 2ull * 2 * 256 * 72 * sizeof(uint16_t);  // 147456 B
  if (lds > d.max_lds) return fail(CATENA_ERR_UNSUPPORTED, "device LDS %zu < %zu", d.max_lds, lds);
  KernelId id = tile_ok ? (out_f32 ? KernelId::GemmBf16TileF32 : KernelId::GemmBf16TileBf16)
                        : (out_f32 ? KernelId::GemmBf16EdgeF32 : KernelId::GemmBf16EdgeBf16);
  return launch(id, dim3((unsigned)tiles), dim3(256), lds, args);
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
  void* args[] = {&q, &k, &v, &lens, &o, &heads, &max_len, &scale};
  // K-pass cache policy: plain loads by default (each 128-byte line of K is
  // read as two halves by consecutive steps and must stay in L2 between
  // them); CATENA_ATTN_K=nt selects the non-temporal form for comparison.
  const char* kp = getenv("CATENA_ATTN_K");
  const bool k_cached = !(kp && strcmp(kp, "nt") == 0);
  return launch(k_cached ? KernelId::AttnDecodeD128KC : KernelId::AttnDecodeD128, dim3((unsigned)bh),
                dim3(256), lds, args);
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
