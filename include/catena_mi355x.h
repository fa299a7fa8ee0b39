/*
 * catena_mi355x.h -- C ABI of the MI355X-native catena hot path.
 *
 * Two layers, both plain C (pointers, sizes, status codes; no torch types):
 *
 *  1. The program ABI that catena's generated module exports and that its
 *     runtime calls through libffi (catena-lang/src/runtime/executor.rs:47-106,
 *     signature table catena-lang/src/runtime/signature.rs:18-72, emitted by
 *     catena-lang/src/codegen/gpu.rs:235-285).  Symbols are
 *     `program_` + the source name with every non-alphanumeric mapped to `_`
 *     (catena-lang/src/codegen/mod.rs:379-388); inputs by value, outputs as
 *     pointers, return void, and assertion / GPU failures are fail-stop
 *     (message on stderr, then a trap: catena-lang/src/codegen/prelude.rs:38-55).
 *
 *  2. The kernel ABI those programs lower to ("catena_mi355x_*"), which
 *     returns a status and never traps, plus the device buffer pool that
 *     replaces the reference's per-buffer managed allocation
 *     (catena-lang/src/runtime/mem.rs:152-171, hipFree on drop :119-125).
 *
 *  3. The runtime mirror ("catena_runtime_*") of Runtime::from_sources /
 *     Runtime::exec / Value (catena-lang/src/runtime/runtime.rs:104-247,
 *     catena-lang/src/runtime/value.rs:5-49).
 *
 * Everything runs on one device and one library-owned HIP stream.  Kernel
 * ABI calls are stream-ordered (asynchronous); program ABI calls and
 * catena_runtime_exec synchronise before returning, like the generated host
 * wrapper (catena-lang/src/codegen/ops/materializec.rs:123-141).
 */
#ifndef CATENA_MI355X_H
#define CATENA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* catena_mem_t: by-value fat pointer, len in BYTES.
 * Reference: catena-lang/src/codegen/prelude.rs:28-31 and
 * catena-lang/src/runtime/executor.rs:14-19 (CatenaMem).  Here `data` is a
 * device pointer owned by the pool; len == 0 means data == NULL
 * (catena-lang/src/codegen/ops/materializec.rs:114). */
typedef struct catena_mem {
  void *data;
  uint64_t len;
} catena_mem_t;

typedef enum catena_status {
  CATENA_OK = 0,
  CATENA_ERR_INVALID_ARGUMENT = 1,
  CATENA_ERR_UNSUPPORTED = 2,
  CATENA_ERR_HIP = 3,
  CATENA_ERR_OUT_OF_MEMORY = 4,
  CATENA_ERR_NOT_INITIALIZED = 5,
  CATENA_ERR_LOAD = 6
} catena_status_t;

/* ------------------------------------------------------------------ */
/* library / device                                                     */

/* Select the device, create the library stream, load the gfx950 code
 * objects (hipModuleLoad) that sit next to this library.  Idempotent.
 * Replaces GpuRuntime::load (catena-lang/src/runtime/mem.rs:134-150) and the
 * per-Runtime hipcc + dlopen of catena-lang/src/runtime/artifact.rs:44-103. */
int catena_mi355x_init(int device);
/* Orderly teardown before the process exits: waits for the library
 * stream, returns the library's own device memory (split-K workspace,
 * completion counters, cached pool blocks), unloads the code objects and
 * destroys the stream.  Buffers the caller still holds stay allocated and
 * may still be freed with catena_mem_free.  A later call re-initialises on
 * demand.  The reference instead keeps its generated library resident for
 * the process lifetime (RTLD_NODELETE, catena-lang/src/runtime/runtime.rs:
 * 249-263); here nothing is left for the runtime's own exit to tear down. */
int catena_mi355x_shutdown(void);
/* Message of the last failing call on this thread ("" if none). */
const char *catena_mi355x_last_error(void);
/* The hipStream_t every launch goes to (for events / interop). */
void *catena_mi355x_stream(void);
int catena_mi355x_synchronize(void);

/* ------------------------------------------------------------------ */
/* device buffer pool                                                    */

/* Allocate len bytes of device memory (size-classed, cached free lists).
 * Replaces Mem allocation (catena-lang/src/runtime/mem.rs:152-171). */
int catena_mem_alloc(uint64_t len, catena_mem_t *out);
/* Return a buffer to the pool and null the handle.  Stream-ordered: work
 * already queued on the library stream may still use it.  Replaces
 * Mem::drop -> hipFree (catena-lang/src/runtime/mem.rs:119-125). */
int catena_mem_free(catena_mem_t *mem);
/* Host <-> device copies (synchronous).  catena_mem_read replaces the raw
 * host dereference of managed memory in Mem::to_f32_vec / to_u64_vec
 * (catena-lang/src/runtime/mem.rs:44-70). */
int catena_mem_write(catena_mem_t mem, uint64_t offset, const void *src, uint64_t len);
int catena_mem_read(catena_mem_t mem, uint64_t offset, void *dst, uint64_t len);
int catena_pool_stats(uint64_t *bytes_live, uint64_t *bytes_cached, uint64_t *device_allocs);
/* Release every cached (free) block back to the device. */
int catena_pool_trim(void);

/* ------------------------------------------------------------------ */
/* kernel ABI (device pointers; stream-ordered)                         */

/* C[n x m] = A[n x k] * B[k x m], f32, row-major, each cell the
 * k-ascending fold acc = acc + A*B from +0.0 with no FMA: bitwise the
 * reference's f32.matmul.row-major.materialize
 * (catena-lang/stdlib/matrix.hex:236-327, lowered by
 * catena-lang/src/codegen/ops/materializec.rs:36-82 and
 * catena-lang/src/codegen/ops/reducec.rs:73-130). */
int catena_mi355x_gemm_f32_exact(const float *a, const float *b, float *c, uint64_t n,
                                 uint64_t m, uint64_t k);

/* C[n x m] = A[n x k] * B[k x m] on bf16 inputs (raw bf16 bits), f32
 * accumulation on MFMA in a fixed order, output bf16 (RNE) or f32 when
 * out_f32 != 0.  Same contraction as above, extended to bf16 (no reference
 * counterpart: catena has no bf16, catena-lang/src/codegen/lower_types.rs:13-22).
 * n <= 16 (decode shape) uses the weight-streaming kernel (both outputs). */
int catena_mi355x_gemm_bf16(const uint16_t *a, const uint16_t *b, void *c, uint64_t n,
                            uint64_t m, uint64_t k, int out_f32);

/* The k split of the decode-shape GEMM (1 <= n <= 16, m % 8 == 0, k % 8 ==
 * 0): the number of k groups whose f32 partials are added in ascending
 * order, and the bytes of those partials (0 when k is not split).  A function
 * of (n, m, k) alone -- never of the device -- so the decode GEMM's bits
 * depend only on the shape and the inputs.  Needs no device.  No reference
 * counterpart (the reference's fold is one sequential chain per cell). */
int catena_mi355x_gemm_bf16_decode_plan(uint64_t n, uint64_t m, uint64_t k, uint32_t *k_groups,
                                        uint64_t *partials_bytes);

/* Allocation-free form of catena_mi355x_gemm_bf16 for decode shapes
 * (1 <= n <= 16, m % 8 == 0, k % 8 == 0, k > 0; 16-byte aligned pointers):
 * the same kernels and the same bits, with the split-K partials in a fixed
 * 4 MiB device array the library holds on each device from load to exit,
 * instead of a workspace it grows with hipMalloc.  No reference counterpart:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc).  Needs a prior
 * catena_mi355x_init (returns CATENA_ERR_NOT_INITIALIZED otherwise; it never
 * initialises, since init allocates); shapes whose partials exceed 4 MiB
 * (see catena_mi355x_gemm_bf16_decode_plan) return CATENA_ERR_UNSUPPORTED.
 * Calls share the device's array: calls that overlap on one device race. */
int catena_mi355x_gemm_bf16_decode_noalloc(const uint16_t *a, const uint16_t *b, void *c,
                                           uint64_t n, uint64_t m, uint64_t k, int out_f32);

/* LM head of a decode step in one launch: c = a * b as the decode shape of
 * catena_mi355x_gemm_bf16 computes it (f32 c[n][m]), and idx[r] =
 * tensor.argmax-f32 of row r of c (catena-lang/stdlib/tensor.hex:204-227:
 * the first maximum after the last NaN, or the last NaN when it is the
 * final element).  1 <= n <= 16, m % 8 == 0, k % 8 == 0, k > 0, m < 2^31,
 * n * ceil(m / 128) <= 57,344 (the per-block summaries' buffer); 16-byte
 * aligned a, b, c.  No reference counterpart (the decoder's greedy step). */
int catena_mi355x_gemm_bf16_argmax(const uint16_t *a, const uint16_t *b, float *c, uint32_t *idx,
                                   uint64_t n, uint64_t m, uint64_t k);

/* Decode attention, one query per (batch, head): q[B][H][D], k/v[B][H][L][D]
 * bf16, lens[B] (device u32, each <= L), o[B][H][D] f32.  Bitwise the
 * sequential composition of cell-dot, nn.softmax and cell-dot
 * (catena-lang/stdlib/matrix.hex:236-256, catena-lang/stdlib/nn.hex:93-122,
 * catena-lang/stdlib/math.hex:148-199).  No reference counterpart (catena
 * has no attention primitive).  head_dim must be 128. */
int catena_mi355x_attn_decode_bf16(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                   const uint32_t *lens, float *o, uint32_t batch,
                                   uint32_t heads, uint32_t max_len, uint32_t head_dim,
                                   float scale);

/* nn.softmax over `rows` contiguous vectors of length n (bitwise the
 * reference's fold order; catena-lang/stdlib/nn.hex:93-122).  y may equal x. */
int catena_mi355x_softmax_f32(const float *x, float *y, uint64_t rows, uint64_t n);

/* math.exp-approx elementwise (catena-lang/stdlib/math.hex:185-199). */
int catena_mi355x_exp_approx_f32(const float *x, float *y, uint64_t n);

/* The scalar stdlib programs elementwise, bitwise the reference's op order
 * (each is one generated __host__ __device__ function in the reference,
 * rendered from these hexpr sources).  y may equal x. */
typedef enum catena_map_op {
  CATENA_MAP_EXP_APPROX = 0,     /* math.exp-approx, catena-lang/stdlib/math.hex:185-199 */
  CATENA_MAP_SQRT = 1,           /* math.sqrt, catena-lang/stdlib/math.hex:235-272 */
  CATENA_MAP_SIGMOID = 2,        /* nn.sigmoid, catena-lang/stdlib/nn.hex:1-12 */
  CATENA_MAP_SILU = 3,           /* nn.silu, catena-lang/stdlib/nn.hex:15-21 */
  CATENA_MAP_SIN_APPROX = 4,     /* math.sin-approx, catena-lang/stdlib/math.hex:1-23 */
  CATENA_MAP_COS_APPROX = 5,     /* math.cos-approx, catena-lang/stdlib/math.hex:25-47 */
  CATENA_MAP_SIN_APPROX_FULL = 6 /* math.sin-approx-full, catena-lang/stdlib/math.hex:49-103 */
} catena_map_op_t;
int catena_mi355x_map_f32(uint32_t op, const float *x, float *y, uint64_t n);

/* Seeded synthetic inputs (counter-based splitmix64; see fill.hip). */
int catena_mi355x_fill_normal_bf16(uint16_t *out, uint64_t n, uint64_t seed, uint64_t stream,
                                   float scale);
int catena_mi355x_fill_uniform_f32(float *out, uint64_t n, uint64_t seed, uint64_t stream);
/* Device-to-device copy kernel (16-byte aligned pointers, n % 16 == 0); also
 * the known-size reference for calibrating HBM traffic counters. */
int catena_mi355x_copy_bytes(void *dst, const void *src, uint64_t n);

/* -- decoder-block pieces (the callers on either side of the two hot ops) -- */

/* Causal KV-cache attention for Tq queries per sequence (prefill, or
 * several tokens per step): q[B][Tq][H][D], k/v[B][H][L][D] bf16,
 * lens[B] (device u32: positions in the cache after the append, <= L),
 * o[B][Tq][H][D] f32 (out_f32 != 0) or bf16 RNE.  Query tq of sequence b
 * attends to the first lens[b] - (Tq - 1 - tq) positions, each exactly as
 * catena_mi355x_attn_decode_bf16 (Tq = 1 is that call).  No reference
 * counterpart.  head_dim must be 128. */
int catena_mi355x_attn_causal_bf16(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                   const uint32_t *lens, void *o, uint32_t batch, uint32_t tq,
                                   uint32_t heads, uint32_t max_len, uint32_t head_dim,
                                   float scale, int out_f32);

/* nn.rmsnorm over `rows` contiguous vectors of length n
 * (catena-lang/stdlib/nn.hex:154-182 with math.sqrt,
 * catena-lang/stdlib/math.hex:235-272): bitwise the reference's fold order.
 * n % 4 == 0; y may not alias x. */
int catena_mi355x_rmsnorm_f32(const float *x, float *y, uint64_t rows, uint64_t n);

/* Residual add in front of nn.rmsnorm, bf16 output: for output row i with
 * src = row_index ? row_index[i] : i, h = x[src] + resid[src] (h = x[src]
 * when resid is NULL), written to h_out[i] when h_out is not NULL; then
 * y[i] = bf16(nn.rmsnorm(h)).  No reference counterpart (the decoder's fused
 * form of f32.add and nn.rmsnorm).  n % 4 == 0. */
int catena_mi355x_residual_rmsnorm_bf16(const float *x, const float *resid,
                                        const uint32_t *row_index, float *h_out, uint16_t *y,
                                        uint64_t rows, uint64_t n);

/* Token embedding: x[r][:] = widen(table[tokens[r]][:]) for r < rows;
 * table[vocab][d] bf16, x f32; a token >= vocab gives a row of NaN.
 * d % 8 == 0.  No reference counterpart. */
int catena_mi355x_embed_bf16(const uint32_t *tokens, const uint16_t *table, float *x,
                             uint64_t rows, uint32_t vocab, uint32_t d);

/* RoPE inverse frequencies on the host: out[i] = (float)(1 / base^(2i/d))
 * in double precision, i < head_dim / 2.  No reference counterpart. */
int catena_mi355x_rope_inv_freq(float *out_host, uint32_t head_dim, double base);

/* RoPE + KV-cache append on a fused projection qkv[B*Tq][3*H*D] f32
 * (columns: q heads | k heads | v heads; row b*Tq + tq at position
 * lens[b] - Tq + tq).  Pairs (i, i + D/2) rotate by theta = pos *
 * inv_freq[i] with sin = math.sin-approx-full
 * (catena-lang/stdlib/math.hex:52-103) and cos the same reduction with the
 * quadrant advanced by one.  Writes q[B*Tq][H*D] bf16 and the bf16 rotated
 * k and v rows into k_cache/v_cache[B][H][L][D].  No reference counterpart. */
int catena_mi355x_rope_qkv_bf16(const float *qkv, const float *inv_freq, const uint32_t *lens,
                                uint16_t *q, uint16_t *k_cache, uint16_t *v_cache,
                                uint32_t batch, uint32_t tq, uint32_t heads, uint32_t head_dim,
                                uint32_t max_len);

/* The rotation table of catena_mi355x_rope_qkv_bf16 for positions 0 ..
 * positions - 1: tab[pos][i] = (cos, sin) of theta = (f32)pos * inv_freq[i],
 * i < head_dim / 2, f32 pairs -- the values that call computes per row.
 * positions <= 65535.  No reference counterpart. */
int catena_mi355x_rope_table_f32(const float *inv_freq, float *tab, uint32_t positions,
                                 uint32_t head_dim);

/* The decoder's prefill q / k / v projection in one kernel:
 * catena_mi355x_gemm_bf16(a, w, qkv, batch * tq, 3 * heads * 128, k, out_f32 = 1)
 * followed by catena_mi355x_rope_qkv_bf16(qkv, ..., head_dim = 128), bitwise,
 * without writing the f32 product.  a[batch * tq][k], w[k][3 * heads * 128]
 * bf16; rope_tab from catena_mi355x_rope_table_f32 with at least max_len
 * positions.  Rows whose position lens[b] - tq + t falls outside [0, max_len)
 * write q (rotated at position 0) and no cache row.  Needs batch * tq % 256
 * == 0, k % 128 == 0, k <= 2^22, 16-byte aligned pointers; other shapes
 * return CATENA_ERR_UNSUPPORTED.  No reference counterpart. */
int catena_mi355x_gemm_bf16_rope_qkv(const uint16_t *a, const uint16_t *w, const float *rope_tab,
                                     const uint32_t *lens, uint16_t *q, uint16_t *k_cache,
                                     uint16_t *v_cache, uint32_t batch, uint32_t tq, uint32_t heads,
                                     uint32_t max_len, uint64_t k);

/* bf16 GEMM as f32 k-split partials (the decoder's prefill W_down):
 * parts[z][n][m] = the product over k in [z k / splits, (z + 1) k / splits),
 * each folded as catena_mi355x_gemm_bf16 folds a product; a consumer adds
 * them in ascending z.  Needs 1 <= splits <= 64, n % 256 == 0, m % 256 == 0,
 * k % (128 splits) == 0, k <= 2^22, 16-byte aligned pointers.  No reference
 * counterpart. */
int catena_mi355x_gemm_bf16_ksplit_f32(const uint16_t *a, const uint16_t *b, float *parts,
                                       uint64_t n, uint64_t m, uint64_t k, uint32_t splits);

/* SwiGLU gate: gu[rows][2F] f32 -> out[rows][F] = bf16(nn.silu(gate) * up)
 * (catena-lang/stdlib/nn.hex:1-21).  group = 0: columns gate | up; group =
 * G: gate and up interleaved in groups of G columns (gate 0..G-1, up
 * 0..G-1, gate G..2G-1, ...), the decoder's W_gu layout (G = 64).
 * F % 4 == 0, G % 4 == 0, F % G == 0.  No reference counterpart. */
int catena_mi355x_silu_mul_bf16(const float *gu, uint16_t *out, uint64_t rows, uint32_t ffn,
                                uint32_t group);

/* bf16 GEMM with the SwiGLU gate fused into its epilogue (the decoder's
 * W_gu projection in prefill): act[n][m/2] = bf16(nn.silu(gate) * up) of the
 * f32 product A[n][k] x B[k][m], whose columns are gate and up interleaved in
 * groups of 64 (catena_mi355x_silu_mul_bf16 with group 64).  Bitwise the same
 * as catena_mi355x_gemm_bf16(..., out_f32 = 1) followed by that call, without
 * writing the f32 product.  Needs the 32-k tile kernels: n % 256 == 0, m % 128
 * == 0, k > 0 with k % 128 == 0, k <= 2^22, m <= 2^24, 16-byte aligned
 * pointers; other shapes return CATENA_ERR_UNSUPPORTED (n == 0 or m == 0 is a
 * no-op).  No reference counterpart. */
int catena_mi355x_gemm_bf16_silu(const uint16_t *a, const uint16_t *b, uint16_t *act, uint64_t n,
                                 uint64_t m, uint64_t k);

/* tensor.argmax-f32 per row (catena-lang/stdlib/tensor.hex:204-227):
 * idx[r] = first index of the maximum with the reference's NaN behaviour;
 * n = 0 gives 0xFFFFFFFF (the reference asserts n != 0). */
int catena_mi355x_argmax_f32(const float *x, uint32_t *idx, uint64_t rows, uint64_t n);

/* -- buffer producers and folds (materializec / reducec programs) -- */

/* tensor.broadcast-f32 body (catena-lang/stdlib/tensor.hex:1-21): out[i] = value. */
int catena_mi355x_broadcast_f32(float *out, uint64_t n, float value);
/* tensor.arange-f32 body (catena-lang/stdlib/tensor.hex:23-46): out[i] =
 * u64.to-f32(i), round to nearest even. */
int catena_mi355x_arange_f32(float *out, uint64_t n);
/* Element copy behind tensor.slice-f32 / tensor.concat-f32
 * (catena-lang/stdlib/tensor.hex:48-168); any 4-byte alignment. */
int catena_mi355x_copy_f32(float *dst, const float *src, uint64_t n);
/* sum-f32 / mean-f32 / max-f32 per row (catena-lang/stdlib/sum.hex:29-101):
 * the reference's sequential folds (sum from +0, max-env from -inf),
 * bitwise.  sum / mean: n <= 0xFFFFF800 (longer rows return
 * CATENA_ERR_UNSUPPORTED); max: n < 2^31. */
int catena_mi355x_sum_f32(const float *x, float *out, uint64_t rows, uint64_t n);
int catena_mi355x_mean_f32(const float *x, float *out, uint64_t rows, uint64_t n);
int catena_mi355x_max_f32(const float *x, float *out, uint64_t rows, uint64_t n);
/* sum-u64 / dot-u64 per row (catena-lang/tests/cases/reducec/basic.hex):
 * wrapping u64 arithmetic. */
int catena_mi355x_sum_u64(const uint64_t *x, uint64_t *out, uint64_t rows, uint64_t n);
int catena_mi355x_dot_u64(const uint64_t *a, const uint64_t *b, uint64_t *out, uint64_t rows,
                          uint64_t n);

/* ------------------------------------------------------------------ */
/* program ABI (generated-module symbols; synchronous; fail-stop)        */

/* tests/cases/matrix/matmul.hex:1-63 "matmul-2x2-via-mem":
 * (mem A, mem B, n, m, k, nk, km, nm) -> (mem C).  Asserts nk == len(A)/4 and
 * km == len(B)/4 like the reference, and additionally n*k == nk, k*m == km,
 * n*m == nm (the reference leaves those to its type checker). */
void program_matmul_2x2_via_mem(catena_mem_t a, catena_mem_t b, uint64_t n, uint64_t m,
                                uint64_t k, uint64_t nk, uint64_t km, uint64_t nm,
                                catena_mem_t *out);
/* tests/cases/matrix/matmul.hex:65-106 / :108-147: A * I and I * A. */
void program_matmul_right_identity_2x2_via_mem(catena_mem_t a, uint64_t n, uint64_t nn,
                                               catena_mem_t *out);
void program_matmul_left_identity_2x2_via_mem(catena_mem_t a, uint64_t n, uint64_t nn,
                                              catena_mem_t *out);
/* catena-lang/stdlib/nn.hex:93-122 "nn.softmax": (mem) -> (mem). */
void program_nn_softmax(catena_mem_t x, catena_mem_t *out);
/* catena-lang/stdlib/math.hex:185-199 "math.exp-approx": (f32) -> (f32). */
void program_math_exp_approx(float x, float *out);
/* The scalar stdlib programs, (f32) -> (f32) each, as the reference's
 * generated module exports them (catena-lang/src/codegen/gpu.rs:235-285):
 *   "math.sqrt"            catena-lang/stdlib/math.hex:235-272
 *   "nn.sigmoid"           catena-lang/stdlib/nn.hex:1-12
 *   "nn.silu"              catena-lang/stdlib/nn.hex:15-21
 *   "math.sin-approx"      catena-lang/stdlib/math.hex:1-23
 *   "math.cos-approx"      catena-lang/stdlib/math.hex:25-47
 *   "math.sin-approx-full" catena-lang/stdlib/math.hex:49-103 */
void program_math_sqrt(float x, float *out);
void program_nn_sigmoid(float x, float *out);
void program_nn_silu(float x, float *out);
void program_math_sin_approx(float x, float *out);
void program_math_cos_approx(float x, float *out);
void program_math_sin_approx_full(float x, float *out);
/* bf16 analogue of matmul-2x2-via-mem (no reference counterpart):
 * (mem A bf16, mem B bf16, n, m, k, nk, km, nm) -> (mem C bf16). */
void program_bf16_matmul_via_mem(catena_mem_t a, catena_mem_t b, uint64_t n, uint64_t m,
                                 uint64_t k, uint64_t nk, uint64_t km, uint64_t nm,
                                 catena_mem_t *out);
/* Decode attention as a program (no reference counterpart):
 * (mem q, mem k, mem v, mem lens u32, batch, heads, max_len, head_dim, f32 scale)
 * -> (mem o f32). */
void program_attn_decode_via_mem(catena_mem_t q, catena_mem_t k, catena_mem_t v,
                                 catena_mem_t lens, uint64_t batch, uint64_t heads,
                                 uint64_t max_len, uint64_t head_dim, float scale,
                                 catena_mem_t *out);

/* catena-lang/stdlib/nn.hex:154-182 "nn.rmsnorm": (mem) -> (mem). */
void program_nn_rmsnorm(catena_mem_t x, catena_mem_t *out);
/* catena-lang/stdlib/tensor.hex:204-227 "tensor.argmax-f32": (mem) -> (u64);
 * traps on an empty input like the reference's u64.assert-nz. */
void program_tensor_argmax_f32(catena_mem_t x, uint64_t *out);

/* catena-lang/stdlib/tensor.hex producers: (f32 value, u64 len) -> (mem);
 * (u64 len) -> (mem); (mem, u64 start, u64 len) -> (mem), trapping unless
 * start + len <= len(input); (mem, mem) -> (mem). */
void program_tensor_broadcast_f32(float value, uint64_t len, catena_mem_t *out);
void program_tensor_arange_f32(uint64_t len, catena_mem_t *out);
void program_tensor_slice_f32(catena_mem_t input, uint64_t start, uint64_t len, catena_mem_t *out);
void program_tensor_concat_f32(catena_mem_t a, catena_mem_t b, catena_mem_t *out);
/* catena-lang/stdlib/sum.hex folds: (mem) -> (f32). */
void program_sum_f32(catena_mem_t x, float *out);
void program_mean_f32(catena_mem_t x, float *out);
void program_max_f32(catena_mem_t x, float *out);
/* catena-lang/tests/cases/reducec/basic.hex: (mem) -> (u64); (mem, mem) ->
 * (u64), trapping unless the lengths are equal. */
void program_sum_u64(catena_mem_t x, uint64_t *out);
void program_dot_u64(catena_mem_t a, catena_mem_t b, uint64_t *out);

/* ------------------------------------------------------------------ */
/* decoder (Llama-style blocks composed from the ops above)              */

/* No reference counterpart: the model the two hot contractions serve.
 * Per layer, rows r of the residual stream x (f32):
 *   xn  = bf16(rmsnorm(x));  qkv = xn * W_qkv (f32);  RoPE + cache append;
 *   o   = bf16(attention);   h = x + o * W_o;  hn = bf16(rmsnorm(h));
 *   gu  = hn * W_gu (f32);   a = bf16(silu(gate) * up);  x' = h + a * W_down.
 * Then bf16(rmsnorm(x)) of each sequence's last row times W_lm gives f32
 * logits and greedy argmax the next token.  Weights bf16, row-major NN:
 * W_qkv[d][3d] (columns q heads | k heads | v heads), W_o[d][d],
 * W_gu[d][2F] (gate and up columns interleaved in groups of 64),
 * W_down[F][d], W_lm[d][vocab]; embedding[vocab][d]. */
typedef struct catena_decoder catena_decoder_t;
typedef struct catena_decoder_config {
  uint32_t d_model;  /* = n_heads * head_dim */
  uint32_t n_heads;
  uint32_t head_dim; /* 128 */
  uint32_t ffn_dim;  /* SwiGLU width F */
  uint32_t n_layers;
  uint32_t vocab;
  uint32_t max_batch; /* <= 4096 */
  uint32_t max_len;   /* cache positions per sequence; the attention holds one
                         f32 score per position in LDS: <= 36,720 on gfx950
                         ((163,840 - 16,960) / 4) */
  float rope_base;
} catena_decoder_config_t;
/* create() rejects (CATENA_ERR_UNSUPPORTED) n_heads or n_layers > 4096,
 * ffn_dim > 2^24, vocab > 2^26, d_model > 20,476 (the RMSNorm holds a row
 * and its squares in LDS: 16 + 8 * d_model <= 163,840 B on gfx950) and the
 * limits above. */

typedef enum catena_decoder_tensor {
  CATENA_DEC_EMBED = 0, /* [vocab][d] bf16 */
  CATENA_DEC_W_QKV,     /* per layer [d][3d] bf16 */
  CATENA_DEC_W_O,       /* per layer [d][d] bf16 */
  CATENA_DEC_W_GU,      /* per layer [d][2F] bf16, gate / up interleaved by 64 */
  CATENA_DEC_W_DOWN,    /* per layer [F][d] bf16 */
  CATENA_DEC_W_LM,      /* [d][vocab] bf16 */
  CATENA_DEC_K_CACHE,   /* per layer [max_batch][H][max_len][D] bf16 */
  CATENA_DEC_V_CACHE,   /* per layer, same */
  CATENA_DEC_INV_FREQ,  /* [D/2] f32 */
  /* activations of the last forward call (rows = batch * tokens per
   * sequence; the last layer's values when n_layers > 1) */
  CATENA_DEC_X,         /* [rows][d] f32: residual stream into the last layer */
  CATENA_DEC_XN,        /* [rows][d] bf16 */
  CATENA_DEC_QKV,       /* [rows][3d] f32; not written by a prefill of rows % 256 == 0
                         * (its projection applies RoPE and fills q and the caches in its
                         * epilogue) */
  CATENA_DEC_Q,         /* [rows][d] bf16 (rotated) */
  CATENA_DEC_ATTN,      /* [rows][d] bf16 */
  CATENA_DEC_ATTN_PROJ, /* [rows][d] f32 */
  CATENA_DEC_H,         /* [rows][d] f32 */
  CATENA_DEC_HN,        /* [rows][d] bf16 */
  CATENA_DEC_GU,        /* [rows][2F] f32, gate / up interleaved by 64; not written by a
                         * prefill of rows % 256 == 0 (the SwiGLU gate runs in the GEMM's
                         * epilogue) */
  CATENA_DEC_ACT,       /* [rows][F] bf16 */
  CATENA_DEC_FFN_OUT,   /* [rows][d] f32; after a prefill whose W_down runs as k-half
                         * partials (rows % 256 == 0, d % 256 == 0, d_ff % 256 == 0, at
                         * most 128 tiles of 256 x 256) only the rows the final norm reads
                         * (each sequence's last) hold the sum */
  CATENA_DEC_FINAL_H,   /* [batch][d] f32: residual stream at the last rows */
  CATENA_DEC_FINAL_XN,  /* [batch][d] bf16 */
  CATENA_DEC_LOGITS,    /* [batch][vocab] f32 */
  CATENA_DEC_LENS,      /* [batch] u32: cache positions per sequence */
  /* [vocab + 1][d] bf16: bf16(rmsnorm(widen(embed[t]))) for every token t,
   * row vocab all NaN (the row of a token out of range); rebuilt by
   * init_weights and, once decoder_tensor(CATENA_DEC_EMBED) has handed out
   * the embedding (which the caller may then write through at any time), at
   * the start of every prefill and generate call (one pass over vocab rows
   * per call, not per step).  A decode step
   * gathers layer 0's normalized input from it, so in a decode step layer
   * 0 writes neither CATENA_DEC_X nor CATENA_DEC_XN. */
  CATENA_DEC_EMBED_NORM,
  CATENA_DEC_TENSOR_COUNT
} catena_decoder_tensor_t;

int catena_mi355x_decoder_create(const catena_decoder_config_t *cfg, catena_decoder_t **out);
void catena_mi355x_decoder_destroy(catena_decoder_t *dec);
/* Device memory owned by the decoder (weights can be written through it). */
int catena_mi355x_decoder_tensor(catena_decoder_t *dec, uint32_t which, uint32_t layer,
                                 catena_mem_t *out);
/* Every weight ~ N(0, std) in bf16 from the seeded counter generator. */
int catena_mi355x_decoder_init_weights(catena_decoder_t *dec, uint64_t seed, float std);
/* Prefill `tokens` (device u32 [batch][t]) into an empty cache, then write
 * each sequence's greedy next token to next (device u32 [batch]). */
int catena_mi355x_decoder_prefill(catena_decoder_t *dec, const uint32_t *tokens,
                                  uint32_t batch, uint32_t t, uint32_t *next);
/* `steps` greedy decode steps after a prefill: step s appends tokens
 * out[s-1] (out[-1] = the prefill's next) and writes out[s][batch].  out is
 * device u32 [steps][batch].  Fails when the cache would overflow. */
int catena_mi355x_decoder_generate(catena_decoder_t *dec, uint32_t steps, uint32_t *out);

/* ------------------------------------------------------------------ */
/* runtime mirror                                                         */

/* ValueKind, catena-lang/src/runtime/value.rs:15-21 */
typedef enum catena_value_kind {
  CATENA_VALUE_BOOL = 0,
  CATENA_VALUE_U32 = 1,
  CATENA_VALUE_U64 = 2,
  CATENA_VALUE_F32 = 3,
  CATENA_VALUE_MEM = 4
} catena_value_kind_t;

/* Value, catena-lang/src/runtime/value.rs:5-12 */
typedef struct catena_value {
  catena_value_kind_t kind;
  union {
    uint8_t b;
    uint32_t u32;
    uint64_t u64;
    float f32;
    catena_mem_t mem;
  } as;
} catena_value_t;

/* ExecError / InitError kinds, catena-lang/src/runtime/runtime.rs:36-102 */
typedef enum catena_exec_status {
  CATENA_EXEC_OK = 0,
  CATENA_EXEC_UNKNOWN_SOURCE_FUNCTION = 1,
  CATENA_EXEC_INPUT_ARITY_MISMATCH = 2,
  CATENA_EXEC_OUTPUT_ARITY_MISMATCH = 3,
  CATENA_EXEC_TYPE_MISMATCH = 4,
  CATENA_INIT_PARSE = 10,
  CATENA_INIT_NO_LOWERING = 11,
  CATENA_INIT_SIGNATURE_MISMATCH = 12,
  CATENA_INIT_DIALECT = 13,
  CATENA_INIT_DEVICE = 14,
  /* not reference error kinds: host memory ran out while reading sources;
   * a NULL runtime, name, source list, argument or output array */
  CATENA_INIT_HOST_MEMORY = 15,
  CATENA_EXEC_BAD_CALL = 20
} catena_exec_status_t;

typedef struct catena_runtime catena_runtime_t;

/* Runtime::from_sources (catena-lang/src/runtime/runtime.rs:115-121).
 * `dialect` is "hip" (the only accepted GpuDialect here).  Sources are
 * scanned for `(def program NAME : TYPE = ...)` forms; every declared
 * program with a native lowering becomes executable, its signature taken
 * from the declared type. */
int catena_runtime_from_sources(const char *const *sources, size_t n_sources,
                                const char *dialect, catena_runtime_t **out);
void catena_runtime_destroy(catena_runtime_t *rt);
/* Runtime::exec (catena-lang/src/runtime/runtime.rs:175-236): validation in
 * the reference's order (unknown name, input arity, output arity, kinds);
 * outputs are written to outs[0..n_outs). */
int catena_runtime_exec(catena_runtime_t *rt, const char *name, const catena_value_t *args,
                        size_t n_args, catena_value_t *outs, size_t n_outs);
/* Details of the last runtime error on this thread (index / expected /
 * actual for TypeMismatch, expected / actual counts for arity errors). */
int catena_runtime_last_error_detail(int64_t *index, int64_t *expected, int64_t *actual);
/* Number of executable programs and their names (for listing). */
size_t catena_runtime_program_count(const catena_runtime_t *rt);
const char *catena_runtime_program_name(const catena_runtime_t *rt, size_t i);
/* Runtime::mem_u64 / mem_f32 (catena-lang/src/runtime/runtime.rs:166-172). */
int catena_runtime_mem_u64(catena_runtime_t *rt, const uint64_t *values, size_t n,
                           catena_value_t *out);
int catena_runtime_mem_f32(catena_runtime_t *rt, const float *values, size_t n,
                           catena_value_t *out);

#ifdef __cplusplus
}
#endif
#endif
