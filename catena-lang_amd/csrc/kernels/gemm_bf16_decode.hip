// Decode-shape bf16 GEMM: Y[M x N] = X[M x K] * W[K x N] for M <= 16, with
// optional fused epilogues for the decoder step.
//
// Same contraction as gemm_bf16.hip (catena-lang/stdlib/matrix.hex:236-327,
// NN row-major, bf16 widened exactly, f32 accumulation) but shaped for the
// decode step, where W dominates the traffic (2*N*K bytes against 2*M*K for
// X) and the kernel is HBM-bound.  All 16 MFMA rows are X's (rows >= M are
// zero), so one v_mfma_f32_16x16x32_bf16 consumes a 32(k) x 16(n) piece of W.
//
// Work split (fixed, data independent):
//   * a workgroup owns 128 consecutive columns and a k range of 4 * KW;
//     its 4 waves each accumulate all 128 columns over part of that range
//     (streaming path: the range's 32-k slabs dealt round robin, wave w
//     taking slabs w, w+4, ...; register path: 4 consecutive chunks of KW),
//     and the workgroup adds the 4 wave sums in wave order through LDS;
//   * grid.y = number of k ranges (S).  With S > 1 each workgroup stores
//     its f32 partial P[s][m][n] (16-byte stores that bypass the XCD caches).
//     Plain outputs (Y f32 or bf16) then end the kernel (EPI_PARTIALS) and
//     catena_decode_reduce, launched next, adds P[0] .. P[S-1] in ascending
//     s.  The fused epilogues instead take a completion ticket for their
//     column block; the last of the S workgroups loads the S partials the
//     same way, adds them in ascending s and runs the epilogue on the final
//     M x 128 tile, staged in LDS.
// The addition order depends only on the shape (which workgroup or launch
// adds never changes how), so results are bitwise identical run to run and
// between the two forms.
//
// Epilogues (each also writes the f32 tile to Y unless EPI_STORE_BF16):
//   EPI_STORE   Y f32;          EPI_STORE_BF16  Y bf16 (RNE)
//   EPI_ROPE    fused q|k|v projection of one decode token per sequence:
//               column block = one head of q, k or v; RoPE + bf16 q out and
//               the K/V cache append, exactly as catena_rope_qkv_store
//   EPI_SILU    SwiGLU with gate / up columns interleaved in groups of 64:
//               act[m][64*bx + c] = bf16(silu(gate) * up), as catena_silu_mul_bf16
//   EPI_PARTIALS  no hand-off: with S > 1 every workgroup stores its partial
//               P[s] and ends, and the kernel that consumes Y adds P[0] ..
//               P[S-1] in ascending s itself (the same adds, so the same
//               bits); the launch boundary orders the partials before that
//               kernel reads them.  With S = 1 it is EPI_STORE.
//   EPI_ARGMAX  LM head: per row, (last NaN, first max) of the block's 128
//               logits as one 16-byte summary, then a second ticket over the
//               column blocks; the last block composes them in column order:
//               tensor.argmax-f32
//               (catena-lang/stdlib/tensor.hex:204-227), as catena_argmax_rows_f32
//
// Streaming (K % 32 == 0): each wave runs a private 4-deep LDS ring of
// [32 k][128 cols] W slabs and [16][32] X slabs filled with direct
// global->LDS loads (nothing held in registers while in flight, so 36 KiB
// per wave are in flight), and reads B fragments with the transposing LDS
// read (no register transpose).  Otherwise (K % 32 != 0): lane l = 16*g + c
// loads the 8x8 block W[k0+8g ..][n0+8c ..] into registers, transposes it
// and feeds column n0+8c+j to MFMA j.
#include "common.h"

namespace {
constexpr int COLS_PER_WAVE = 128;
constexpr int TILE_LD = 132;  // f32 row stride of the LDS output tile

enum Epi : int { EPI_STORE = 0, EPI_STORE_BF16 = 1, EPI_ROPE = 2, EPI_SILU = 3, EPI_ARGMAX = 4, EPI_PARTIALS = 5 };

CATENA_DEV bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

CATENA_DEV void transpose8x8(const u32x4_t in[8], u32x4_t out[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      uint32_t x = in[2 * p][j / 2], y = in[2 * p + 1][j / 2];
      w[p] = (j & 1) ? ((x >> 16) | (y & 0xFFFF0000u)) : ((x & 0xFFFFu) | (y << 16));
    }
    out[j] = u32x4_t{w[0], w[1], w[2], w[3]};
  }
}

CATENA_DEV void load_w(const uint16_t* __restrict__ W, uint64_t K, uint64_t N, uint64_t k0,
                       uint64_t col, int g, u32x4_t r[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint64_t kr = k0 + 8 * g + i;
    if (kr < K && col < N)
      r[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(W + kr * N + col));
    else
      r[i] = u32x4_t{0u, 0u, 0u, 0u};
  }
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;

// LDS ring of the streaming path: per wave RING stages, each a W slab
// [32 k][128 cols] (8 KiB, 256-byte rows) and an X slab [16 rows][32 k]
// (1 KiB, chunks swizzled by row bits 1-2).  16-byte chunk p of W row r holds global chunk p ^ hW(r), which
// makes the transposing fragment reads (16 rows x 32 bytes per
// instruction) hit every bank pair once.
constexpr int RING = 4;
constexpr int W_SLAB = 32 * 128 * 2;
constexpr int STAGE_BYTES = W_SLAB + 1024;
constexpr int WAVE_RING = RING * STAGE_BYTES;
CATENA_DEV uint32_t hW(uint32_t r) { return 2u * ((r & 3u) | (((r >> 3) & 1u) << 2)); }

CATENA_DEV bf16x8_t cat_bf16(i16x4_t lo, i16x4_t hi) {
  typedef short i16x8_t __attribute__((ext_vector_type(8)));
  i16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8_t, v);
}

// Buffer descriptor word 3 for raw (unswizzled, stride 0) 32-bit access, and
// the cache-policy operand that sets sc1: the encoding the compiler uses for
// agent-scope atomic loads and stores, which bypass the XCD-private caches.
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kCpolSc1 = 16;

// s_waitcnt on vmcnt only (gfx9 encoding: vmcnt[3:0], vmcnt[5:4] at 15:14)
#define DEC_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | 0x0070 | 0x0F00)

}  // namespace

// Extra operands of the fused epilogues (unused fields may be null).
struct DecodeEpi {
  // EPI_ROPE
  uint16_t* q_out;          // [M][H*128] bf16
  uint16_t* k_cache;        // [B][H][L][128]
  uint16_t* v_cache;
  const uint32_t* lens;     // [M] positions after the append
  const float* inv_freq;    // [64]
  uint32_t heads, max_len;
  // EPI_SILU
  uint16_t* act;            // [M][N/2] bf16
  // EPI_ARGMAX
  uint32_t* idx;            // [M]
  uint32_t* arg_ticket;     // one counter, zero between launches
  uint32_t* arg_partials;   // [M][gridDim.x][4]: last NaN, max value, max index, pad
  // row m of X is X[min(x_rows[m], x_rows_limit)] when x_rows is given (a
  // gather from a table whose row x_rows_limit is the out-of-range row)
  const uint32_t* x_rows;
  uint32_t x_rows_limit;
  // EPI_ROPE: (cos, sin) of every (position, pair), [max_len][64][2], when
  // given (the values cos_full / sin_full give, so the same bits)
  const float* rope_tab;
  // X rows by tokens composed here from a deferred LM-head argmax: when
  // x_sums is given, row m's token is the argmax of row m of those column-
  // block summaries ([M][x_sums_blocks][4], over x_sums_cols logits), and
  // workgroup (0, 0) writes the M tokens to x_rows_out
  const uint32_t* x_sums;
  uint32_t x_sums_blocks;
  uint64_t x_sums_cols;
  uint32_t* x_rows_out;
  // EPI_ARGMAX: nonzero -> only the logits and the summaries are written;
  // the argmax is composed by the next kernel that needs it
  uint32_t arg_defer;
};

// Argmax composition from per-column-block summaries (u32x4: last NaN or
// -1, first-max bits, first-max column or 0xFFFFFFFF, pad) of one row, in
// column order, by one wave: the last NaN J* is the largest J; the answer is
// the first maximum over the blocks from J*'s block on, whose summaries hold
// their first maximum after their own last NaN (after J* in J*'s block, over
// the whole block after it) -- the first maximum as the largest (monotone
// value, complemented column) pair -- or J* itself if it is the last column.
// Summaries are loaded coherently (sc1); pe holds the row's first 256 (lane
// l: blocks l, l + 64, l + 128, l + 192), loaded by argmax_first_sums.
// (loaded from an in-range block and replaced past gx, so that no branch
// sits around the load and waits for it can leave later loads in flight)
CATENA_DEV u32x4_t argmax_sum_load(__amdgpu_buffer_rsrc_t ars, uint32_t r, uint32_t gx, uint32_t b) {
  const u32x4_t v =
      __builtin_amdgcn_raw_buffer_load_b128(ars, (int)(((uint64_t)r * gx + (b < gx ? b : gx - 1)) * 16), 0, kCpolSc1);
  return b < gx ? v : u32x4_t{0xFFFFFFFFu, 0u, 0xFFFFFFFFu, 0u};
}
// (raw loads: the blocks past gx are replaced in argmax_compose, so nothing
// waits on these loads until it runs)
CATENA_DEV void argmax_first_sums(__amdgpu_buffer_rsrc_t ars, uint32_t r, uint32_t gx, uint32_t lane,
                                  u32x4_t (&pe)[4]) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint32_t b = lane + 64u * u;
    pe[u] = __builtin_amdgcn_raw_buffer_load_b128(ars, (int)(((uint64_t)r * gx + (b < gx ? b : gx - 1)) * 16), 0,
                                                  kCpolSc1);
  }
}
CATENA_DEV uint32_t argmax_compose(__amdgpu_buffer_rsrc_t ars, uint32_t r, uint32_t gx, uint64_t N,
                                   uint32_t lane, const u32x4_t (&pe_raw)[4]) {
  u32x4_t pe[4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
    pe[u] = lane + 64u * u < gx ? pe_raw[u] : u32x4_t{0xFFFFFFFFu, 0u, 0xFFFFFFFFu, 0u};
  uint32_t jm = 0, bm = 0, bl = 0;  // J + 1; best monotone value, its complemented column
  auto take = [&](uint32_t b, const u32x4_t& pv, uint32_t bstart) {
    if (b < gx && b >= bstart && pv[2] != 0xFFFFFFFFu) {
      const uint32_t mo = mono_bits(pv[1]), lo = (0x7FFFFFFFu - pv[2]) << 1;
      if (mo > bm || (mo == bm && lo > bl)) {
        bm = mo;
        bl = lo;
      }
    }
  };
#pragma unroll
  for (int u = 0; u < 4; ++u) jm = pe[u][0] + 1u > jm ? pe[u][0] + 1u : jm;
  for (uint32_t b0 = 256; b0 < gx; b0 += 256)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const u32x4_t pv = argmax_sum_load(ars, r, gx, b0 + lane + 64u * u);
      jm = pv[0] + 1u > jm ? pv[0] + 1u : jm;
    }
  const uint32_t J1 = wave_umax(jm);  // J* + 1, 0 when no NaN
  const uint32_t bstart = J1 ? (J1 - 1) / 128u : 0u;
#pragma unroll
  for (int u = 0; u < 4; ++u) take(lane + 64u * u, pe[u], bstart);
  for (uint32_t b0 = 256; b0 < gx; b0 += 256)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t b = b0 + lane + 64u * u;
      take(b, argmax_sum_load(ars, r, gx, b), bstart);
    }
  const uint32_t M_hi = wave_umax(bm);
  const uint32_t L_lo = wave_umax(bm == M_hi ? bl : 0u);
  return (J1 != 0u && J1 == N) ? (uint32_t)(N - 1) : 0x7FFFFFFFu - (L_lo >> 1);
}
// Rows r = wave, wave + 4, ... < M of a 4-wave workgroup, two rows per pass
// with both rows' summary loads in flight together; out(r, idx) from lane 0.
template <typename Out>
CATENA_DEV void argmax_compose_rows(__amdgpu_buffer_rsrc_t ars, uint32_t M, uint32_t gx, uint64_t N,
                                    uint32_t wave, uint32_t lane, Out out) {
  for (uint32_t r = wave; r < M; r += 8) {
    const bool two = r + 4 < M;
    u32x4_t pa[4], pb[4];
    argmax_first_sums(ars, r, gx, lane, pa);
    argmax_first_sums(ars, two ? r + 4 : r, gx, lane, pb);
    const uint32_t ia = argmax_compose(ars, r, gx, N, lane, pa);
    if (lane == 0) out(r, ia);
    if (two) {
      const uint32_t ib = argmax_compose(ars, r + 4, gx, N, lane, pb);
      if (lane == 0) out(r + 4, ib);
    }
  }
}

template <int EPI, int WAUX>
CATENA_DEV void decode_body(const uint16_t* __restrict__ X, const uint16_t* __restrict__ W,
                            void* __restrict__ Y, float* __restrict__ P,
                            uint32_t* __restrict__ tickets, uint32_t M, uint64_t N, uint64_t K,
                            uint32_t KW, uint32_t stream_lds, const DecodeEpi& ep) {
  // Dynamic LDS: the streaming ring, reused after the k loop for the four
  // waves' sums (red[4][8][64]) and the output tile.
  extern __shared__ __attribute__((aligned(1024))) unsigned char dsm[];
  f32x4_t(*red)[8][64] = reinterpret_cast<f32x4_t(*)[8][64]>(dsm);
  float* tile = reinterpret_cast<float*>(dsm + 4 * 8 * 64 * 16);
  __shared__ uint32_t last_flag;
  const bool streamed = stream_lds != 0;  // host: only when K % 32 == 0

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const uint64_t n0 = (uint64_t)blockIdx.x * COLS_PER_WAVE;
  const uint64_t col = n0 + 8 * c;
  const uint64_t kbeg = ((uint64_t)blockIdx.y * 4 + wave) * KW;
  uint64_t kend = kbeg + KW;
  if (kend > K) kend = K;

  f32x4_t acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  if (streamed) {
    // Streaming path: W and X slabs go global -> LDS (global_load_lds, no
    // registers held by loads in flight) through this wave's RING-deep
    // ring; B fragments are read with the transposing LDS read, so lane
    // (G, s) of MFMA block j gets W[k0 + 8G .. +7][n0 + 16j + s].  Output:
    // lane (G, s) holds rows 4G .. 4G+3 of column n0 + 16j + s.
    unsigned char* ring = dsm + wave * WAVE_RING;
    // The workgroup's k range [kg0, kg1) is dealt to its waves in 32-k
    // slabs, round robin (wave w takes slabs w, w+4, ...), so the four
    // streams cover neighbouring rows of W and finish together.
    const uint64_t kg0 = (uint64_t)blockIdx.y * 4 * KW;
    uint64_t kg1 = kg0 + 4ull * KW;
    if (kg1 > K) kg1 = K;
    const uint32_t nslab = kg0 < kg1 ? (uint32_t)((kg1 - kg0) / 32) : 0u;
    const uint32_t steps = nslab > (uint32_t)wave ? (nslab - (uint32_t)wave + 3u) / 4u : 0u;
    const uint64_t kw0 = kg0 + 32ull * wave;
    // per-lane global byte offsets of the 8 W instructions (4 rows each)
    // (a lane whose columns lie past N reads the block's first columns
    // instead: every load is issued, so the per-stage waits count exactly,
    // and those columns' sums are never stored)
    uint32_t woff[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t r = 4 * i + (lane >> 4);
      const uint32_t q = (uint32_t)(lane & 15) ^ hW(r);
      const bool live = n0 + 8 * q < N;
      woff[i] = (uint32_t)(((uint64_t)r * N + (live ? 8 * q : 0u)) * 2);
    }
    // X slab: lane l fetches row l / 4 into slot l % 4, which holds the
    // row's global chunk (l % 4) ^ ((row >> 1) & 3): the fragment read
    // (lane 16 G + s: row s, chunk G) is then free of LDS bank conflicts
    // (measured with SQ_LDS_BANK_CONFLICT; unswizzled it costs 8 LDS cycles
    // per read instead of 4)
    const uint32_t xr = lane >> 2, xq = (uint32_t)(lane & 3) ^ ((xr >> 1) & 3u);
    const bool xl = xr < M;
    const char* wsrc = reinterpret_cast<const char*>(W) + (kw0 * N + n0) * 2;
    // W's cache policy (WAUX, 2 = non-temporal).  A non-temporal stream
    // reads faster (a long read on gfx950: 7.1 against 6.1 TB/s; the C3
    // shapes 21.2 -> 20.4 and 20.7 -> 19.3 us per call) but leaves nothing
    // in the Infinity Cache: the plain-output kernels and the LM head
    // (argmax), whose weights are read once, use it; the decode step's
    // block projections do not, so that the cache keeps the block weights
    // and the KV cache between steps (C5 decode step 94.6 us against 104.9
    // with every weight stream non-temporal).
    constexpr int kWAux = WAUX;
    auto issue_w = [&](uint32_t t, int slot) {  // slab t of this wave = k kw0 + 128 t
      unsigned char* st = ring + slot * STAGE_BYTES;
      const char* w = wsrc + (uint64_t)t * 128 * N * 2;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        __builtin_amdgcn_global_load_lds(w + woff[i], (lds_void*)(st + 1024 * i), 16, 0, kWAux);
    };
    const uint32_t pre = steps < (uint32_t)RING ? steps : (uint32_t)RING;
    uint32_t xrow = xr;
    if (ep.x_sums) {
      // the tokens of the previous step's LM head, composed from its column
      // block summaries (the same composition its own last workgroup makes)
      __shared__ uint32_t tok_s[16];
      const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
          (void*)ep.x_sums, (short)0, (int)((uint64_t)M * ep.x_sums_blocks * 16), kRsrcWord3);
      argmax_compose_rows(srs, M, ep.x_sums_blocks, ep.x_sums_cols, (uint32_t)wave, (uint32_t)lane,
                          [&](uint32_t r, uint32_t idx) { tok_s[r] = idx; });
      __syncthreads();
      if (blockIdx.x == 0 && blockIdx.y == 0 && tid < (int)M) ep.x_rows_out[tid] = tok_s[tid];
      if (xl) {
        xrow = tok_s[xr];
        if (xrow > ep.x_rows_limit) xrow = ep.x_rows_limit;
      }
    } else if (ep.x_rows && xl) {
      xrow = ep.x_rows[xr];
      if (xrow > ep.x_rows_limit) xrow = ep.x_rows_limit;
    }
    // rows past M read row 0: loaded, never stored (an MFMA output row
    // depends on its own A row only), so every X request is issued too
    if (!xl) xrow = 0;
    const char* xsrc = reinterpret_cast<const char*>(X) + ((uint64_t)xrow * K + kw0 + 8 * xq) * 2;
    auto issue_x = [&](uint32_t t, int slot) {
      __builtin_amdgcn_global_load_lds(xsrc + (uint64_t)t * 256, (lds_void*)(ring + slot * STAGE_BYTES + W_SLAB), 16,
                                       0, 0);
    };
    auto issue = [&](uint32_t t, int slot) {
      issue_w(t, slot);
      issue_x(t, slot);
    };
    for (uint32_t t = 0; t < pre; ++t) issue(t, (int)t);
    // fragment read addresses inside a stage
    const int G = lane >> 4, sl = lane & 15;
    const uint32_t xa_off = W_SLAB + ((uint32_t)sl * 4 + ((uint32_t)G ^ (((uint32_t)sl >> 1) & 3u))) * 16;
    const uint32_t brow = 8 * G + (sl >> 2);
    const uint32_t hb = hW(brow);
    uint32_t b_off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t colq = 16 * j + 4 * (sl & 3);
      b_off[j] = brow * 256 + 16 * ((colq >> 3) ^ hb) + 2 * (colq & 7);
    }
    for (uint32_t t = 0; t < steps; ++t) {
      const int slot = (int)(t % RING);
      const uint32_t later = steps - 1 - t < (uint32_t)(RING - 1) ? steps - 1 - t : (uint32_t)(RING - 1);
      // every instruction of stage t has landed; the later stages may not
      // have (9 instructions per stage)
      if (later >= 3) {
        DEC_WAIT_VMCNT(27);
      } else if (later == 2) {
        DEC_WAIT_VMCNT(18);
      } else if (later == 1) {
        DEC_WAIT_VMCNT(9);
      } else {
        DEC_WAIT_VMCNT(0);
      }
      asm volatile("" ::: "memory");
      const unsigned char* st = ring + slot * STAGE_BYTES;
      const bf16x8_t af = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(st + xa_off));
      bf16x8_t bf[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const unsigned char* pb = st + b_off[j];
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(pb));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(pb + 4 * 256));
        bf[j] = cat_bf16(lo, hi);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf[j], acc[j], 0, 0, 0);
      if (t + RING < steps) {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this slot's reads are done
        asm volatile("" ::: "memory");
        issue(t + RING, slot);
      }
    }
  } else {
    const int xr16 = lane & 15;
    const bool xlive = xr16 < (int)M;
    uint64_t xrow = (uint64_t)xr16;
    if (ep.x_rows && xlive) {
      xrow = ep.x_rows[xr16];
      if (xrow > ep.x_rows_limit) xrow = ep.x_rows_limit;
    }
    if (kbeg < kend) {
      u32x4_t cur[8], nxt[8];
      load_w(W, K, N, kbeg, col, g, cur);
      for (uint64_t k0 = kbeg; k0 < kend; k0 += 32) {
        const bool more = k0 + 32 < kend;
        if (more) load_w(W, K, N, k0 + 32, col, g, nxt);
        const uint64_t xk = k0 + 8 * g;
        u32x4_t xa = u32x4_t{0u, 0u, 0u, 0u};
        if (xlive && xk < K) xa = *reinterpret_cast<const u32x4_t*>(X + xrow * K + xk);
        u32x4_t bt[8];
        transpose8x8(cur, bt);
        const bf16x8_t af = as_bf16x8(xa);
#pragma unroll
        for (int j = 0; j < 8; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, as_bf16x8(bt[j]), acc[j], 0, 0, 0);
        if (more) {
#pragma unroll
          for (int i = 0; i < 8; ++i) cur[i] = nxt[i];
        }
      }
    }
  }
  // the streaming path's LDS is reused below
  __syncthreads();

  // every wave's sums into LDS; then all threads add the four waves' values
  // of each f32x4 in wave order, ((w0 + w1) + w2) + w3, into the tile (lane
  // (G, s) of register j holds rows 4G .. 4G+3 of tile column 16j + s when
  // streamed, else 8s + j)
#pragma unroll
  for (int j = 0; j < 8; ++j) red[wave][j][lane] = acc[j];
  __syncthreads();
  for (uint32_t e = tid; e < 8u * 64u; e += 256) {
    const uint32_t j = e >> 6, ln = e & 63u;
    f32x4_t v = red[0][j][ln];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const f32x4_t o = red[w][j][ln];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = v[q] + o[q];
    }
    const uint32_t gg = ln >> 4, sc = ln & 15u;
    const uint32_t tc = streamed ? 16 * j + sc : 8 * sc + j;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t row = 4 * gg + q;
      if (row < M) tile[row * TILE_LD + tc] = v[q];
    }
  }
  __syncthreads();
  const uint32_t S = gridDim.y;
  if (S > 1) {
    // This workgroup's partial, P[blockIdx.y][m][n0 ..], read by another
    // workgroup: 16-byte stores that bypass the XCD-private caches (sc1), as
    // agent-scope atomics do, from all threads.
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)P, (short)0, (int)(S * (uint64_t)M * N * 4), kRsrcWord3);
    for (uint32_t e = tid; e < M * 32u; e += 256) {
      const uint32_t row = e >> 5, c4 = 4 * (e & 31u);
      if (n0 + c4 < N) {
        const float* t = tile + row * TILE_LD + c4;
        const u32x4_t v = u32x4_t{__float_as_uint(t[0]), __float_as_uint(t[1]),
                                  __float_as_uint(t[2]), __float_as_uint(t[3])};
        __builtin_amdgcn_raw_buffer_store_b128(
            v, prs, (int)((((uint64_t)blockIdx.y * M + row) * N + n0 + c4) * 4), 0, kCpolSc1);
      }
    }
    if (EPI == EPI_PARTIALS) return;
    if (!last_arrival(&tickets[blockIdx.x], S, &last_flag)) return;
    // Last k group of this column block: P[0] + P[1] + ... + P[S-1],
    // ascending s, for the block's M rows x 128 columns; every partial's
    // 16-byte coherent load of a batch (16 partials) is issued before the
    // adds.
    for (uint32_t e = tid; e < M * 32u; e += 256) {
      const uint32_t row = e >> 5, c4 = 4 * (e & 31u);
      const uint64_t cc = n0 + c4;
      f32x4_t sum = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if (cc < N) {
        const uint64_t base = ((uint64_t)row * N + cc) * 4, MN4 = (uint64_t)M * N * 4;
        for (uint32_t s0 = 0; s0 < S; s0 += 16) {
          u32x4_t part[16];
#pragma unroll
          for (int u = 0; u < 16; ++u)
            if (s0 + u < S)
              part[u] = __builtin_amdgcn_raw_buffer_load_b128(prs, (int)(base + (s0 + u) * MN4), 0, kCpolSc1);
#pragma unroll
          for (int u = 0; u < 16; ++u)
            if (s0 + u < S) {
              if (s0 + u == 0) {
#pragma unroll
                for (int q = 0; q < 4; ++q) sum[q] = __uint_as_float(part[u][q]);
              } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) sum[q] = sum[q] + __uint_as_float(part[u][q]);
              }
            }
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) tile[row * TILE_LD + c4 + q] = sum[q];
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- epilogue
  // tile[m][0..127] holds Y[m][n0 .. n0+127]
  for (uint32_t e = tid; e < M * 32u; e += 256) {
    const uint32_t row = e >> 5, c4 = 4 * (e & 31u);
    const uint64_t cc = n0 + c4;
    if (cc >= N) continue;
    const float* t = tile + row * TILE_LD + c4;
    if (EPI == EPI_STORE_BF16) {
      uint2 o;
      o.x = pack_bf16x2(t[0], t[1]);
      o.y = pack_bf16x2(t[2], t[3]);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(Y) + (uint64_t)row * N + cc) = o;
    } else if (EPI == EPI_ARGMAX) {
      // the logits go past the XCD cache (sc1), so the completion ticket's
      // release below has no dirty lines of them to write back
      const __amdgpu_buffer_rsrc_t yrs =
          __builtin_amdgcn_make_buffer_rsrc(Y, (short)0, (int)((uint64_t)M * N * 4), kRsrcWord3);
      const u32x4_t v = u32x4_t{__float_as_uint(t[0]), __float_as_uint(t[1]), __float_as_uint(t[2]),
                                __float_as_uint(t[3])};
      __builtin_amdgcn_raw_buffer_store_b128(v, yrs, (int)(((uint64_t)row * N + cc) * 4), 0, kCpolSc1);
    } else {
      *reinterpret_cast<f32x4_t*>(static_cast<float*>(Y) + (uint64_t)row * N + cc) =
          f32x4_t{t[0], t[1], t[2], t[3]};
    }
  }

  if (EPI == EPI_ROPE) {
    // column block = (part, head): part 0 q, 1 k, 2 v; one token per row
    const uint32_t H = ep.heads, L = ep.max_len;
    const uint32_t part = blockIdx.x / H, head = blockIdx.x % H;
    const uint64_t HD = (uint64_t)H * 128;
    for (uint32_t e = tid; e < M * 64u; e += 256) {
      const uint32_t r = e >> 6, i = e & 63u;
      const uint32_t len = ep.lens[r];
      const bool pos_ok = len >= 1 && len - 1 < L;
      const uint32_t pos = pos_ok ? len - 1 : 0u;
      const float* t = tile + r * TILE_LD;
      const uint64_t cache = (((uint64_t)r * H + head) * L + pos) * 128;
      if (part == 2) {
        if (pos_ok) {
          ep.v_cache[cache + i] = (uint16_t)f32_to_bf16_bits(t[i]);
          ep.v_cache[cache + i + 64] = (uint16_t)f32_to_bf16_bits(t[i + 64]);
        }
        continue;
      }
      float cs, sn;
      if (ep.rope_tab) {
        const float2 cp = reinterpret_cast<const float2*>(ep.rope_tab)[(uint64_t)pos * 64 + i];
        cs = cp.x;
        sn = cp.y;
      } else {
        const float pf = (float)pos;
        const float theta = pf * ep.inv_freq[i];
        cs = cos_full(theta);
        sn = sin_full(theta);
      }
      const float x1 = t[i], x2 = t[i + 64];
      const float t1 = x1 * cs, t2 = x2 * sn, t3 = x2 * cs, t4 = x1 * sn;
      const float y1 = t1 - t2, y2 = t3 + t4;
      if (part == 0) {
        uint16_t* dq = ep.q_out + (uint64_t)r * HD + (uint64_t)head * 128;
        dq[i] = (uint16_t)f32_to_bf16_bits(y1);
        dq[i + 64] = (uint16_t)f32_to_bf16_bits(y2);
      } else if (pos_ok) {
        ep.k_cache[cache + i] = (uint16_t)f32_to_bf16_bits(y1);
        ep.k_cache[cache + i + 64] = (uint16_t)f32_to_bf16_bits(y2);
      }
    }
  }

  if (EPI == EPI_SILU) {
    const uint64_t F = N / 2;
    for (uint32_t e = tid; e < M * 64u; e += 256) {
      const uint32_t r = e >> 6, cidx = e & 63u;
      const float* t = tile + r * TILE_LD;
      const float act = silu_approx(t[cidx]);
      const float a = act * t[64 + cidx];
      ep.act[(uint64_t)r * F + 64ull * blockIdx.x + cidx] = (uint16_t)f32_to_bf16_bits(a);
    }
  }

  if (EPI == EPI_ARGMAX) {
    const uint32_t gx = gridDim.x;
    const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
        (void*)ep.arg_partials, (short)0, (int)((uint64_t)M * gx * 16), kRsrcWord3);
    // this block's summary of row r (lane l holds columns n0 + l and
    // n0 + 64 + l): the last NaN from two ballots, then the first maximum
    // after it as the largest monotone value (DPP max; every value that is
    // not NaN has a nonzero one) and the lowest column holding it (ballots)
    // -- the first_max_combine result.  Branch-free, so a wave's two rows
    // (r, r + 4) run as one straight sequence whose ballots, DPP steps and
    // readlanes overlap.
    auto summary = [&](uint32_t r) -> u32x4_t {
      const float* t = tile + r * TILE_LD;
      const float v0 = t[lane], v1 = t[lane + 64];
      const bool in0 = n0 + lane < N, in1 = n0 + 64 + lane < N;
      const uint64_t nan0 = __builtin_amdgcn_ballot_w64(in0 && v0 != v0);
      const uint64_t nan1 = __builtin_amdgcn_ballot_w64(in1 && v1 != v1);
      const int J = nan1 != 0u   ? (int)(n0 + 64 + (63u - (uint32_t)__builtin_clzll(nan1)))
                    : nan0 != 0u ? (int)(n0 + (63u - (uint32_t)__builtin_clzll(nan0)))
                                 : -1;
      const uint32_t b0 = __float_as_uint(v0), b1 = __float_as_uint(v1);
      const uint32_t m0 = (in0 && v0 == v0 && (int)(n0 + lane) > J) ? mono_bits(b0) : 0u;
      const uint32_t m1 = (in1 && v1 == v1 && (int)(n0 + 64 + lane) > J) ? mono_bits(b1) : 0u;
      const uint32_t m = wave_umax(m0 > m1 ? m0 : m1);
      const uint64_t w0 = __builtin_amdgcn_ballot_w64(m != 0u && m0 == m);
      const uint64_t w1 = __builtin_amdgcn_ballot_w64(m != 0u && m1 == m);
      const int wl = w0 != 0u ? __builtin_ctzll(w0) : w1 != 0u ? __builtin_ctzll(w1) : 0;
      const uint32_t fb = (uint32_t)__builtin_amdgcn_readlane((int)(w0 != 0u ? b0 : b1), wl);
      // empty (no value after the last NaN): -inf, no index
      const uint32_t fv = m != 0u ? fb : 0xFF800000u;
      const uint32_t fi = m == 0u ? 0xFFFFFFFFu : (uint32_t)(n0 + (w0 != 0u ? 0u : 64u) + (uint32_t)wl);
      return u32x4_t{(uint32_t)J, fv, fi, 0u};
    };
    for (uint32_t r = wave; r < M; r += 8) {
      const bool two = r + 4 < M;
      const u32x4_t sa = summary(r), sb = summary(two ? r + 4 : r);
      if (lane == 0) {
        // 16-byte summaries, stored past the XCD caches (sc1)
        __builtin_amdgcn_raw_buffer_store_b128(sa, ars, (int)(((uint64_t)r * gx + blockIdx.x) * 16), 0,
                                               kCpolSc1);
        if (two)
          __builtin_amdgcn_raw_buffer_store_b128(sb, ars, (int)(((uint64_t)(r + 4) * gx + blockIdx.x) * 16),
                                                 0, kCpolSc1);
      }
    }
    if (ep.arg_defer) return;
    // the last column block composes every row's argmax from the summaries
    if (!last_arrival(ep.arg_ticket, gx, &last_flag)) return;
    argmax_compose_rows(ars, M, gx, N, (uint32_t)wave, (uint32_t)lane,
                        [&](uint32_t r, uint32_t idx) { ep.idx[r] = idx; });
  }
}

// grid = (ceil(N/128), S), block = 256.  KW = k per wave (multiple of 32).
// tickets[ceil(N/128)] start at zero and are left at zero.
#define CATENA_DECODE_KERNEL(NAME, EPI, WAUX)                                                    \
  extern "C" __global__ __launch_bounds__(256) void NAME(                                        \
      const uint16_t* __restrict__ X, const uint16_t* __restrict__ W, void* __restrict__ Y,     \
      float* __restrict__ P, uint32_t* __restrict__ tickets, uint32_t M, uint64_t N, uint64_t K, \
      uint32_t KW, uint32_t stream_lds, DecodeEpi ep) {                                          \
    decode_body<EPI, WAUX>(X, W, Y, P, tickets, M, N, K, KW, stream_lds, ep);                    \
  }

// plain outputs (the decode GEMM entry point): W non-temporal
CATENA_DECODE_KERNEL(catena_gemm_bf16_decode_f32out, EPI_STORE, 2)
CATENA_DECODE_KERNEL(catena_gemm_bf16_decode_bf16out, EPI_STORE_BF16, 2)
CATENA_DECODE_KERNEL(catena_gemm_bf16_decode_parts_nt, EPI_PARTIALS, 2)
// the decoder's step
CATENA_DECODE_KERNEL(catena_gemm_bf16_decode_rope, EPI_ROPE, 0)
CATENA_DECODE_KERNEL(catena_gemm_bf16_decode_silu, EPI_SILU, 0)
CATENA_DECODE_KERNEL(catena_gemm_bf16_decode_argmax, EPI_ARGMAX, 2)
CATENA_DECODE_KERNEL(catena_gemm_bf16_decode_parts, EPI_PARTIALS, 0)

// The split-K reduction of a plain decode GEMM, as a launch of its own after
// the partials kernel (catena_gemm_bf16_decode_parts_nt): Y = ((P[0] + P[1]) + ...) + P[S-1]
// elementwise, ascending s -- the adds the last-arriving workgroup of the
// ticketed form makes, so the same bits -- stored as f32 or as bf16 (RNE).
// The launch boundary orders the partials before these loads, which takes
// the place of the ticket's agent-scope release / acquire (an L2 write-back
// per workgroup and an L2 invalidate per column block).  Four elements per
// thread; n4 = M * N / 4.
extern "C" __global__ __launch_bounds__(256) void catena_decode_reduce(const float* __restrict__ P,
                                                                       uint64_t part_elems, uint32_t S,
                                                                       void* __restrict__ Y, uint64_t n4,
                                                                       uint32_t out_bf16) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const f32x4_t* p4 = reinterpret_cast<const f32x4_t*>(P) + i;
  const uint64_t st4 = part_elems / 4;
  f32x4_t sum = p4[0];
  for (uint32_t s0 = 1; s0 < S; s0 += 8) {
    f32x4_t v[8];
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u)
      if (s0 + u < S) v[u] = p4[(s0 + u) * st4];
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u)
      if (s0 + u < S) {
#pragma unroll
        for (int q = 0; q < 4; ++q) sum[q] = sum[q] + v[u][q];
      }
  }
  if (out_bf16) {
    uint2 o;
    o.x = pack_bf16x2(sum[0], sum[1]);
    o.y = pack_bf16x2(sum[2], sum[3]);
    reinterpret_cast<uint2*>(Y)[i] = o;
  } else {
    reinterpret_cast<f32x4_t*>(Y)[i] = sum;
  }
}

// The argmax of a deferred LM head (arg_defer): idx[m] composed from the M
// rows of gx column-block summaries over N logits.  One 256-thread
// workgroup.
extern "C" __global__ __launch_bounds__(256) void catena_argmax_compose(const uint32_t* __restrict__ sums,
                                                                        uint32_t M, uint32_t gx, uint64_t N,
                                                                        uint32_t* __restrict__ idx) {
  const __amdgpu_buffer_rsrc_t srs =
      __builtin_amdgcn_make_buffer_rsrc((void*)sums, (short)0, (int)((uint64_t)M * gx * 16), kRsrcWord3);
  argmax_compose_rows(srs, M, gx, N, threadIdx.x >> 6, threadIdx.x & 63u,
                      [&](uint32_t r, uint32_t v) { idx[r] = v; });
}
