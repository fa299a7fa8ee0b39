// Internal declarations shared by the host-side translation units of
// libcatena_mi355x (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>

#include "catena_mi355x.h"

namespace catena {

enum class KernelId : int {
  GemmF32Exact = 0,
  GemmF32ExactT16,  // 16x16 tiles for small outputs (gemm_f32_exact.hip)
  GemmF32ExactQ16,  // 16x16 tiles, A by DPP row broadcast: k % 16 == 0, m % 4 == 0
  GemmBf16EdgeBf16,  // general shapes, bounds-checked (gemm_bf16.hip)
  GemmBf16EdgeF32,
  GemmBf16LdsBf16,  // aligned tiles with K % 128 != 0: two 64-k stages (gemm_bf16_lds.hip)
  GemmBf16LdsF32,
  GemmBf16K32Bf16,  // four 32-k stages, spread buffer loads, LDS-staged epilogue (default)
  GemmBf16K32F32,
  GemmBf16K32N128Bf16,  // the same on 256 x 128 tiles
  GemmBf16K32N128F32,
  GemmBf16K32Silu,  // the 32-k kernels with the SwiGLU epilogue
  GemmBf16K32N128Silu,
  GemmBf16K32N128Rope,  // the 256 x 128 tile kernel with the RoPE + cache epilogue
  GemmBf16K32F32Parts,  // 256 x 256 tiles, k split over grid.y, f32 partials
  GemmBf16DecodeF32,
  GemmBf16DecodeBf16,
  GemmBf16DecodeRope,
  GemmBf16DecodeSilu,
  GemmBf16DecodeArgmax,
  GemmBf16DecodeParts,
  GemmBf16DecodePartsNt,
  ArgmaxCompose,
  DecodeReduce,
  AttnDecodeD128,
  AttnFewD128F32,  // eight waves per pair for few pairs (attn_few.hip)
  AttnFewD128Bf16,
  AttnFewSplitD128F32,  // two seven-wave workgroups per pair (attn_few.hip)
  AttnFewSplitD128Bf16,
  AttnCausalD128F32,
  AttnCausalD128Bf16,
  AttnPrefillD128F32,
  AttnPrefillD128Bf16,
  EmbedRowsBf16,
  RmsnormRows,
  RopeQkvStore,
  RopeTable,
  SiluMulBf16,
  ArgmaxRowsF32,
  BroadcastF32,
  ArangeF32,
  CopyF32,
  SumRowsF32,
  MaxRowsF32,
  SumRowsU64,
  SoftmaxRows,
  ExpApprox,
  MapF32,
  FillNormalBf16,
  FillUniformF32,
  Copy16,
  Count
};

struct Device {
  // set (release) once init has finished; read (acquire) by every entry point
  std::atomic<bool> ready{false};
  // held from workspace() through the launch that uses it, so no thread can
  // launch with a block another thread is replacing
  std::mutex ws_mu;
  int device = -1;
  hipStream_t stream = nullptr;
  size_t max_lds = 0;
  int cu_count = 0;
  hipFunction_t fn[static_cast<int>(KernelId::Count)] = {};
  // code objects loaded at init (unloaded by catena_mi355x_shutdown)
  static constexpr int kMaxModules = 32;
  hipModule_t modules[kMaxModules] = {};
  int n_modules = 0;
  void* ws = nullptr;  // split-K partials
  uint64_t ws_bytes = 0;
  // Zeroed once at init; kernels that take completion tickets return their
  // counters to zero.  Layout: kTicketsGemm column-block counters,
  // kTicketsRows row counters, kTicketsMisc single counters, then
  // kRowPartialBytes of per-row partials.
  unsigned char* small = nullptr;
  static constexpr uint32_t kTicketsGemm = 16384;
  static constexpr uint32_t kTicketsRows = 16384;
  static constexpr uint32_t kTicketsMisc = 256;
  static constexpr uint64_t kRowPartialBytes = 896 * 1024;
  static constexpr uint64_t kSmallBytes =
      4ull * (kTicketsGemm + kTicketsRows + kTicketsMisc) + kRowPartialBytes;
  uint32_t* gemm_tickets() const { return reinterpret_cast<uint32_t*>(small); }
  uint32_t* row_tickets() const { return gemm_tickets() + kTicketsGemm; }
  uint32_t* misc_tickets() const { return row_tickets() + kTicketsRows; }
  void* row_partials() const { return misc_tickets() + kTicketsMisc; }
};

// LDS of the one-query attention kernels (attn_decode.hip): q in f32, the
// K / V staging area, reduction slots, then one f32 score per position.
constexpr size_t kAttnLdsFixed = 128 * 4 + 16384 + 64;
inline size_t attn_lds_bytes(uint32_t max_len) { return kAttnLdsFixed + (size_t)max_len * 4; }

// The eight-wave attention (attn_few.hip) for few (query, head) pairs, where
// the four-wave kernel leaves CUs idle or underfed: one workgroup per pair,
// at most one per CU.  LDS: six q copies and the max words, 64 KiB for the
// six 4 KiB K stages and later the two product slots, two 40 KiB V rings
// (148 KiB), then 64 f32 scores per 64-row block.
constexpr uint64_t kAttnFewMaxQueries = 256;
constexpr size_t kAttnFewFixed = 4096 + 2 * 32768 + 2 * 5 * 8192;
inline size_t attn_few_lds_bytes(uint32_t max_len) {
  return kAttnFewFixed + (size_t)((max_len + 63) / 64) * (64 * 4);
}
// The split form (up to 128 pairs, so at most 256 workgroups): two
// seven-wave workgroups per pair, each with one column half's product
// slots and V ring (77,824 B fixed).
constexpr uint64_t kAttnFewSplitMaxQueries = 128;
constexpr size_t kAttnFewSplitFixed = 4096 + 2 * 16384 + 5 * 8192;
inline size_t attn_few_split_lds_bytes(uint32_t max_len) {
  return kAttnFewSplitFixed + (size_t)((max_len + 63) / 64) * (64 * 4);
}
// A decode step's q / k / v as its fused projection's k-group partials
// (FewQkv in attn_few.hip, field for field): parts[n_parts][rows][3 H 128]
// f32, added in ascending order, q / k rotated with rope_tab
// ([max_len][64] (cos, sin)), q written to q_out (bf16), the sums to qkv_out
// (when given) and the new k / v rows to k_cache / v_cache at lens[b] - 1.
struct FewQkvArgs {
  const float* parts = nullptr;
  uint64_t part_stride = 0;
  uint32_t n_parts = 0;
  const float* rope_tab = nullptr;
  uint16_t* q_out = nullptr;
  float* qkv_out = nullptr;
  uint16_t* k_cache = nullptr;
  uint16_t* v_cache = nullptr;
};
// Whether the eight-wave attention serves this shape.
bool attn_few_fits(uint32_t batch, uint32_t tq, uint32_t heads, uint32_t max_len);
// catena_mi355x_attn_causal_bf16 for a caller that knows every lens[b] <=
// len_bound: the prefill kernel's score buffer is sized for len_bound
// instead of max_len (the decoder's prefill: lens = t)
int attn_causal(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint32_t* lens,
                void* o, uint32_t batch, uint32_t tq, uint32_t heads, uint32_t max_len,
                uint32_t len_bound, uint32_t head_dim, float scale, int out_f32);
// Launch the eight-wave attention when it applies; returns -1 (nothing
// launched) when it does not.
int attn_few_launch(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint32_t* lens,
                    void* o, uint32_t batch, uint32_t tq, uint32_t heads, uint32_t max_len,
                    float scale, bool out_f32, const FewQkvArgs& qkv = FewQkvArgs());

// LDS of catena_rmsnorm_rows (block.hip): its static __shared__ f32 (rounded
// up to the 16-byte alignment of the dynamic area that follows it) plus the
// dynamic row of h and of its squares, n rounded up to a multiple of 4.
constexpr size_t kRmsnormLdsStatic = 16;
inline size_t rmsnorm_lds_bytes(uint64_t n) {
  return kRmsnormLdsStatic + 2 * ((n + 3) & ~3ull) * sizeof(float);
}

Device& device();
int ensure_init();
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
const char* last_error();
int hip_check(hipError_t e, const char* what);
int launch(KernelId id, dim3 grid, dim3 block, size_t lds, void** args);
int pool_alloc(uint64_t len, void** out);
int pool_free(void* ptr);
uint64_t pool_capacity(void* ptr);
int workspace(uint64_t bytes, void** out);

// Extra operands of the fused decode-GEMM epilogues; layout shared with
// struct DecodeEpi in gemm_bf16_decode.hip (passed by value as a kernel
// argument).
struct DecodeEpiArgs {
  uint16_t* q_out = nullptr;
  uint16_t* k_cache = nullptr;
  uint16_t* v_cache = nullptr;
  const uint32_t* lens = nullptr;
  const float* inv_freq = nullptr;
  uint32_t heads = 0, max_len = 0;
  uint16_t* act = nullptr;
  uint32_t* idx = nullptr;
  uint32_t* arg_ticket = nullptr;
  uint32_t* arg_partials = nullptr;
  // X row m = X[min(x_rows[m], x_rows_limit)] when x_rows is not null
  const uint32_t* x_rows = nullptr;
  uint32_t x_rows_limit = 0;
  // Rope: (cos, sin) of every (position, pair) when not null
  // ([max_len][64][2] f32, rope_table_f32), else computed
  const float* rope_tab = nullptr;
  // X rows by the tokens of a deferred argmax: row m = X[min(argmax of row m
  // of x_sums, x_rows_limit)], x_sums being a deferred LM head's summaries
  // ([n][x_sums_blocks][4] u32 over x_sums_cols logits); the tokens are also
  // written to x_rows_out
  const uint32_t* x_sums = nullptr;
  uint32_t x_sums_blocks = 0;
  uint64_t x_sums_cols = 0;
  uint32_t* x_rows_out = nullptr;
  // Argmax: nonzero -> write the logits and the summaries (to arg_partials
  // when given) only, for a later x_sums gather or argmax_compose
  uint32_t arg_defer = 0;
};
enum class DecodeEpilogue { StoreF32, StoreBf16, Rope, Silu, Argmax, Partials };
// Decode-shape GEMM (n <= 16) with an epilogue; c is Y (f32, or bf16 for
// StoreBf16).  Rope: m = 3 * heads * 128, one token per row; Silu: gate / up
// interleaved in 64-column groups, act[n][m/2]; Argmax: idx[n].  The split-K
// partials go to `scratch` (scratch_bytes long) when it is not NULL, else to
// the library's pool-backed workspace.  whole_k: every workgroup streams the
// whole K of its column block (no k groups, partials or ticket), for weights
// that stay in the Infinity Cache between calls, where the hand-off costs
// more than spreading K over more CUs gains (K % 32 == 0 only).
int gemm_bf16_decode(const uint16_t* a, const uint16_t* b, void* c, uint64_t n, uint64_t m,
                     uint64_t k, DecodeEpilogue epi, const DecodeEpiArgs& ep,
                     void* scratch = nullptr, uint64_t scratch_bytes = 0, bool whole_k = false);
// Bytes of split-K partials the decode GEMM needs for an (n x k) * (k x m)
// product (0 when K is not split), and its number of k groups; a function of
// the shape alone.
uint64_t decode_partials_bytes(uint64_t n, uint64_t m, uint64_t k, uint32_t* k_groups);
// The decode GEMM without its split-K hand-off: writes the product's S k-group
// partials parts[s][n][m] (f32; S = *k_groups, parts[0] = the product when
// S = 1) for a consumer that adds them in ascending s.  parts_bytes must hold
// max(S, 1) * n * m floats.
// idx[m] = the argmax of row m of a deferred LM head's summaries
// ([n][blocks][4] u32 over cols logits), as its own composition would give.
int argmax_compose(const uint32_t* sums, uint32_t n, uint32_t blocks, uint64_t cols, uint32_t* idx);
int gemm_bf16_decode_parts(const uint16_t* a, const uint16_t* b, float* parts, uint64_t parts_bytes,
                           uint64_t n, uint64_t m, uint64_t k, uint32_t* k_groups,
                           const DecodeEpiArgs& gather = DecodeEpiArgs());
// Scratch of the allocation-free decode GEMM (noalloc.hip): its device
// address, looked up once per device at init (noalloc_setup, with that
// device current), and its size.
int noalloc_setup(int device);
void* noalloc_scratch(int device);
uint64_t noalloc_scratch_bytes();

// Whether catena_mi355x_gemm_bf16_silu takes this shape (the 32-k tile
// kernels: n % 256, m % 128, k % 128 == 0, aligned operands).
bool gemm_bf16_silu_fits(uint64_t n, uint64_t m, uint64_t k, const void* a, const void* b,
                         const void* act);
// Fused q / k / v projection of a prefill: rows x (3 heads 128) from a
// k-deep bf16 input and weight, then RoPE (the rotation read from tab,
// [positions][64][2] cos / sin), bf16 q [rows][heads 128] and the K / V cache
// rows [batch][heads][max_len][128] at pos = lens[b] - tq + t -- the bits of
// catena_mi355x_gemm_bf16 followed by catena_mi355x_rope_qkv_bf16, without
// the f32 product.  gemm_bf16_rope_fits says whether the 256 x 128 tile
// kernel takes the shape (rows % 256 == 0, rows % tq == 0, k % 128 == 0,
// 16-byte aligned operands).
bool gemm_bf16_rope_fits(uint64_t rows, uint64_t k, uint32_t tq, uint32_t heads, const void* a,
                         const void* w, const void* q_out, const void* kc, const void* vc,
                         const void* tab);
// f32 partials of a k-split GEMM on 256 x 256 tiles: parts[z] [n][m] for
// z < splits, split z folding k in [z k / splits, (z + 1) k / splits); the
// consumer adds them in ascending z.  gemm_bf16_ksplit_fits: n % 256 == 0,
// m % 256 == 0, k % (128 splits) == 0, aligned operands.
bool gemm_bf16_ksplit_fits(uint64_t n, uint64_t m, uint64_t k, uint32_t splits, const void* a,
                           const void* b, const void* parts);
int gemm_bf16_f32_ksplit(const uint16_t* a, const uint16_t* b, float* parts, uint64_t n, uint64_t m,
                         uint64_t k, uint32_t splits);
int gemm_bf16_rope_qkv(const uint16_t* a, const uint16_t* w, const float* tab, const uint32_t* lens,
                       uint16_t* q_out, uint16_t* kc, uint16_t* vc, uint64_t rows, uint64_t k,
                       uint32_t tq, uint32_t heads, uint32_t max_len);
// nn.rmsnorm rows whose input is an embedding gather (x = widen(table[tok]))
// written to x_out, bf16 output.
int embed_rmsnorm_bf16(const uint32_t* tokens, const uint16_t* table, uint32_t vocab,
                       float* x_out, uint16_t* y, uint64_t rows, uint64_t n);
// The same with a residual: h = widen(table[tok]) + resid to h_out, bf16
// rmsnorm(h) to y.
int embed_residual_rmsnorm_bf16(const uint32_t* tokens, const uint16_t* table, uint32_t vocab,
                                const float* resid, float* h_out, uint16_t* y, uint64_t rows,
                                uint64_t n, uint32_t resid_parts = 1, float* resid_out = nullptr);
// h = x[src] + resid[src] and y = bf16(rmsnorm(h)) where resid arrives as
// resid_parts k-group partials of resid_rows x n floats each (added in
// ascending order, the sum also written to resid_out when given); src =
// row_index ? row_index[row] : row.
int residual_parts_rmsnorm_bf16(const float* x, const float* resid, uint32_t resid_parts,
                                float* resid_out, const uint32_t* row_index, float* h_out,
                                uint16_t* y, uint64_t rows, uint64_t resid_rows, uint64_t n);
// bf16 rmsnorm(widen(table[t])) for every t < vocab into y[t], and a row of
// NaN at y[vocab] (the row of a token out of range).
int embed_norm_table_bf16(const uint16_t* table, uint32_t vocab, uint16_t* y, uint64_t n);
// tab[pos][i] = (cos, sin) of (f32)pos * inv_freq[i] for pos < positions,
// i < half, as the RoPE kernels compute them.
int rope_table_f32(const float* inv_freq, float* tab, uint32_t positions, uint32_t half);

// Fail-stop used by the program ABI: message on stderr, then trap, like
// catena_assert / catena_host_gpu_check (catena-lang/src/codegen/prelude.rs:38-55).
[[noreturn]] void trap_assert(const char* what);
[[noreturn]] void trap_gpu(const char* what);

}  // namespace catena
