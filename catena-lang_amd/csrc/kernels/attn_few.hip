// KV-cache attention for few (query, head) pairs -- the decode step of a
// small batch -- in one kernel of eight waves per pair, so that each pair's
// positions and output columns spread over more of its CU than the
// four-wave kernel of attn_decode.hip manages.  Same definition and fold
// orders as attn_decode.hip, so the same bits:
//   s_t = (fold_{d asc} from +0 of q_d * k_{t,d}) * scale
//         -- f32.matmul.cell-dot order, catena-lang/stdlib/matrix.hex:236-256
//   m   = f32.max-env fold from -inf        (catena-lang/stdlib/sum.hex:73-84)
//   den = f32.add-env fold from +0 of exp~(s_t - m)  (catena-lang/stdlib/nn.hex:93-114)
//   p_t = exp~(s_t - m) / den                (catena-lang/stdlib/nn.hex:75-90)
//   o_d = fold_{t asc} from +0 of p_t * v_{t,d}
//
// Layouts as attn_decode.hip: q[B][Tq][H][128], k/v[B][H][L][128] bf16,
// lens[B], o[B][Tq][H][128] f32 or bf16; workgroup qi = (b * Tq + tq) * H + h
// attends to the first lens[b] - (Tq - 1 - tq) positions (clamped to L).
//
// Waves 0-5 score: each first requests its own copy of q, then all four
// 32-wide d segments of its first two 64-row blocks (blocks w, w+6, ...;
// coalesced 16-byte loads, 4 lanes per 64-byte row segment), and folds each
// segment through its LDS slice with lane l owning row l (one d-ascending
// chain of v_mul_f32 + v_add_f32 per score).  The max fold is reduced with
// one LDS atomic per wave and block for each of the last NaN position and a
// 64-bit key whose maximum is the first maximal score (see max_key).  When a NaN precedes the
// last position the key is taken again over the positions after it.  Then
// every score wave computes exp~ for its share of positions, wave 0 runs the
// denominator (the one sequential chain), and the score waves divide their
// shares.
// Waves 6 and 7 own output columns 0-63 and 64-127.  Once the score waves
// have requested their K rows (so that K, which is needed first, is ahead
// of V in the memory queues) they stream their V rows (128 bytes per row)
// straight into LDS rings of 64-row batches.  Once p is ready the batches
// go through rounds separated by workgroup barriers: in round b the score
// waves make batch b + 1's rounded products p_t * v_{t,c} into one of two
// product slots (16 units of 8 rows x 64 columns) while waves 6 and 7
// add batch b's products from the other slot, lane = column, t ascending,
// and refill the ring slot batch b came from.
//
// Cost (measured on MI355X): a wave that runs alone on its SIMD issues an
// instruction about every 4-5 cycles whatever its kind, so a fold that
// unpacks, multiplies and adds per position and column in the same wave,
// with its ring bookkeeping, took about 25 cycles per position.  Split this
// way, the adding waves issue one v_add_f32 and a quarter of a 16-byte LDS
// read per position, and the multiplies run on all four SIMDs.
#include "common.h"

namespace {
constexpr int D = 128;
constexpr int KWAVES = 6;
constexpr int KSTAGE_ROW = 64;                // bytes per staged row segment
constexpr int KSTAGE_WAVE = 64 * KSTAGE_ROW;  // 4096 B per wave
CATENA_DEV uint32_t kswz(uint32_t row, uint32_t chunk) { return 16u * (chunk ^ ((row >> 2) & 3u)); }

constexpr int VB_ROWS = 64;              // rows per V batch
constexpr int VB_BYTES = VB_ROWS * 128;  // 64 rows x 64 columns bf16
constexpr int VRING = 5;                 // batches in flight per V wave (8 loads each)
constexpr int HALF_PSLOT = 64 * 64 * 4;  // one batch's products of one column half

// LDS: q copies [6][128] f32 | den, last score, last NaN, max keys | new key
// row | K stages [6][4 KiB] until the scores are done, then the product
// slots [2][NH][HALF_PSLOT] | V rings [NH][VRING][8 KiB] | scores
// sp[64 * ceil(L/64)], with NH = 2 column halves per workgroup, or 1 in the
// split form (two workgroups per pair, one column half each)
constexpr uint32_t kOffDen = KWAVES * 512;
constexpr uint32_t kOffKNew = kOffDen + 256;  // the new key row (partials mode), 256 B
constexpr uint32_t kOffK = 4096;
constexpr uint32_t kOffP = 4096;
template <int NH>
struct FewLayout {
  static constexpr uint32_t PSLOT = NH * HALF_PSLOT;
  static constexpr uint32_t OffV = kOffP + 2 * PSLOT;
  static constexpr uint32_t OffState = OffV + NH * VRING * VB_BYTES;
  static_assert(kOffK + KWAVES * KSTAGE_WAVE <= OffV, "K stages inside the product slots' space");
};

CATENA_DEV void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations, not for its global loads (the V waves' requests stay in
// flight through the barriers).
CATENA_DEV void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt on vmcnt only (gfx9 encoding: vmcnt[3:0], vmcnt[5:4] at 15:14)
#define FEW_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | 0x0070 | 0x0F00)
// s_waitcnt on lgkmcnt only (bits 11:8), pinned in place by scheduling
// barriers so that the reads and adds around it keep their order
#define FEW_WAIT_LGKM(n)                                   \
  do {                                                     \
    __builtin_amdgcn_sched_barrier(0);                     \
    __builtin_amdgcn_s_waitcnt(0xC07F | ((n) << 8));       \
    __builtin_amdgcn_sched_barrier(0);                     \
  } while (0)

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) unsigned char lds_u8;
typedef __attribute__((address_space(3))) f32x4_t lds_f32x4;

// Lane j of each 16-lane row broadcast to its row (DPP row_newbcast); j is a
// constant once the callers' loops are unrolled.
CATENA_DEV float row_bcast(float x, int j) {
#define CATENA_ROW_BCAST(J) \
  case J:                   \
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x150 + J, 0xF, 0xF, false))
  switch (j) {
    CATENA_ROW_BCAST(0); CATENA_ROW_BCAST(1); CATENA_ROW_BCAST(2); CATENA_ROW_BCAST(3);
    CATENA_ROW_BCAST(4); CATENA_ROW_BCAST(5); CATENA_ROW_BCAST(6); CATENA_ROW_BCAST(7);
    CATENA_ROW_BCAST(8); CATENA_ROW_BCAST(9); CATENA_ROW_BCAST(10); CATENA_ROW_BCAST(11);
    CATENA_ROW_BCAST(12); CATENA_ROW_BCAST(13); CATENA_ROW_BCAST(14); default: break;
  }
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x15F, 0xF, 0xF, false));
#undef CATENA_ROW_BCAST
}

}  // namespace

// A decode step's q / k / v as the k-group partials of its fused projection
// (parts != null; Tq = 1, row = b): the kernel adds them in ascending k group
// (the adds the projection's own reduction makes), rotates q and k with the
// RoPE table rows of the row's position pos = lens[b] - 1 (the rotation the
// projection's epilogue makes), rounds to bf16, writes q_out, the f32 sums
// to qkv_out (when given) and the new k / v rows to the caches at pos (when
// pos < L), and attends with them: the new key's row is put into the
// registers of the block that holds it and the new value's row into its V
// batch in LDS, so the rows read from the caches at pos are never used.
struct FewQkv {
  const float* parts;    // [n_parts][rows][3 * H * 128]
  uint64_t part_stride;  // rows * 3 * H * 128
  uint32_t n_parts;
  const float* rope_tab;  // [L][64] (cos, sin) pairs
  uint16_t* q_out;        // [rows][H * 128]
  float* qkv_out;         // [rows][3 * H * 128] or null
  uint16_t* k_cache;      // the caches k / v read, written at pos
  uint16_t* v_cache;
};

namespace {

// SPLIT: two workgroups per pair (grid = 2 x pairs, 7 waves each): both
// make all the scores and the softmax, workgroup half hf (the upper half of
// the grid) adds output columns 64 hf .. 64 hf + 63 with its one V wave.
// The same operands in the same order, so the same bits; in partials mode
// both write the same q, k and f32 sums (identical values), each its half
// of the new value row.
template <bool OUT_BF16, bool SPLIT>
CATENA_DEV void attn_few_body(const uint16_t* __restrict__ q, const uint16_t* k, const uint16_t* v,
                              const uint32_t* __restrict__ lens, void* __restrict__ o, uint32_t H, uint32_t L,
                              uint32_t Tq, float scale, const FewQkv& qkv) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  typedef FewLayout<SPLIT ? 1 : 2> Lay;
  constexpr uint32_t PSLOT_BYTES = Lay::PSLOT, kOffV = Lay::OffV, kOffState = Lay::OffState;
  float* den_slot = reinterpret_cast<float*>(smem + kOffDen);
  float* last_slot = den_slot + 1;                                          // score at len - 1
  uint32_t* nan_word = reinterpret_cast<uint32_t*>(smem + kOffDen + 8);     // last NaN + 1
  uint64_t* key_word = reinterpret_cast<uint64_t*>(smem + kOffDen + 16);    // [2] max keys
  float* sp = reinterpret_cast<float*>(smem + kOffState);  // 16-byte aligned

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t qi = blockIdx.x, hf = 0;
  if (SPLIT) {
    const uint32_t np = gridDim.x / 2;
    hf = blockIdx.x >= np ? 1u : 0u;
    qi = blockIdx.x - hf * np;
  }
  const uint32_t row = qi / H, h = qi % H;
  const uint32_t b = row / Tq, tq = row % Tq;
  uint32_t len = lens[b];
  if (len > L) len = L;
  const uint32_t later = Tq - 1 - tq;
  len = len > later ? len - later : 0u;
  const uint64_t bh = (uint64_t)b * H + h;
  const uint16_t* kb = k + bh * (uint64_t)L * D;
  const uint16_t* vb = v + bh * (uint64_t)L * D;
  const uint32_t nblk = (len + 63u) / 64u;
  // partials mode: the new row's position and the sum of a column's parts
  const uint32_t raw_len = lens[b];
  const bool pos_ok = raw_len >= 1u && raw_len - 1u < L;
  const uint32_t pos = pos_ok ? raw_len - 1u : 0u;
  const uint64_t HD = (uint64_t)H * D;
  // Columns c and c2 of the fused row, parts added in ascending order, in
  // two steps so that callers can put other loads between them: part_loads
  // issues the first four parts' loads, part_sums adds them (and loads and
  // adds any further parts).
  struct PartLoads {
    uint64_t c, c2;
    float v[4], v2[4];
  };
  auto part_loads = [&](uint64_t c, uint64_t c2, PartLoads& pl) {
    const float* p = qkv.parts + (uint64_t)row * 3 * HD;
    const uint32_t n = qkv.n_parts;
    pl.c = c;
    pl.c2 = c2;
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) {
      const uint64_t o = (u < n ? u : 0u) * qkv.part_stride;
      pl.v[u] = p[o + c];
      pl.v2[u] = p[o + c2];
    }
  };
  auto part_sums = [&](const PartLoads& pl, float& x, float& x2) {
    const float* p = qkv.parts + (uint64_t)row * 3 * HD;
    const uint32_t n = qkv.n_parts;
    x = pl.v[0];
    x2 = pl.v2[0];
#pragma unroll
    for (uint32_t u = 1; u < 4; ++u) {  // (selects, not branches: one straight sequence)
      const float s1 = x + pl.v[u], s2 = x2 + pl.v2[u];
      x = u < n ? s1 : x;
      x2 = u < n ? s2 : x2;
    }
    for (uint32_t u = 4; u < n; ++u) {
      x = x + p[u * qkv.part_stride + pl.c];
      x2 = x2 + p[u * qkv.part_stride + pl.c2];
    }
  };
  // pair (lane, lane + 64) of head h's part 0 (q) or 1 (k): rope_loads
  // issues its loads, rope_pair adds the parts and rotates,
  // y1 = x1 c - x2 s, y2 = x2 c + x1 s (each op rounded)
  struct RopeLoads {
    PartLoads pl;
    float2 cp;
  };
  auto rope_loads = [&](uint32_t part, RopeLoads& rl) {
    const uint64_t c0 = part * HD + (uint64_t)h * D + (uint32_t)lane;
    rl.cp = reinterpret_cast<const float2*>(qkv.rope_tab)[(uint64_t)pos * 64 + (uint32_t)lane];
    part_loads(c0, c0 + 64, rl.pl);
  };
  auto rope_pair = [&](const RopeLoads& rl, float& x1, float& x2, float& y1, float& y2) {
    part_sums(rl.pl, x1, x2);
    const float t1 = x1 * rl.cp.x, t2 = x2 * rl.cp.y, t3 = x2 * rl.cp.x, t4 = x1 * rl.cp.y;
    y1 = t1 - t2;
    y2 = t3 + t4;
  };

  if (wave >= KWAVES) {
    // ---------------------------------------------------------- V waves
    const uint32_t vw = (uint32_t)wave - KWAVES;  // this workgroup's column half
    const uint32_t colbase = 64u * (SPLIT ? hf : vw);
    // the ring's LDS offset, uniform across the wave (so M0 is set from a
    // scalar register)
    const uint32_t ring_off = __builtin_amdgcn_readfirstlane(kOffV + vw * (VRING * VB_BYTES));
    // batch bt -> slot bt % VRING: 8 direct-to-LDS loads of 1 KiB (8 rows x
    // 128 bytes; lane l: row l / 8, chunk l % 8).  In the last batch rows
    // past len read row 0 instead (in bounds, never folded), so every batch
    // is exactly 8 loads and the waits below are exact.  V is read with the
    // non-temporal hint (cache policy nt): in the C5 decode step that keeps
    // more of the weights in the Infinity Cache and measured 19.1 -> 18.6 us
    // for this kernel.
    const uint32_t vr = (uint32_t)lane >> 3, vc = (uint32_t)lane & 7u;
    const uint16_t* vlane = vb + (uint64_t)vr * D + colbase + 8 * vc;
    // partials mode: this wave's column of the new value row, to the cache
    // and into its V batch once that batch is in LDS; its parts' loads go
    // out now, the sum is taken once the first V batches are requested
    const bool new_val = qkv.parts && pos_ok;
    uint16_t vnew = 0;
    PartLoads vpl;
    if (qkv.parts) {
      const uint64_t cv = 2 * HD + (uint64_t)h * D + colbase + (uint32_t)lane;
      part_loads(cv, cv, vpl);
    }
    const uint32_t bt_new = pos / (uint32_t)VB_ROWS;
    auto put_new_val = [&](uint32_t bt) {
      if (new_val && bt == bt_new) {
        uint16_t* slot16 = reinterpret_cast<uint16_t*>(smem + ring_off + (bt % VRING) * VB_BYTES);
        slot16[(pos % VB_ROWS) * 64 + lane] = vnew;
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): written before any lane reads it
        __builtin_amdgcn_wave_barrier();
      }
    };
    auto issue = [&](uint32_t bt) {
      unsigned char* slot = smem + ring_off + (bt % VRING) * VB_BYTES;
      if ((bt + 1) * VB_ROWS <= len) {
        const uint16_t* src = vlane + (uint64_t)bt * VB_ROWS * D;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          __builtin_amdgcn_global_load_lds(src + 8 * i * D, (lds_void*)(slot + 1024 * i), 16, 0, 2);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          uint32_t t = bt * VB_ROWS + 8 * i + vr;
          if (t >= len) t = 0;
          __builtin_amdgcn_global_load_lds(vb + (uint64_t)t * D + colbase + 8 * vc,
                                           (lds_void*)(slot + 1024 * i), 16, 0, 2);
        }
      }
    };
    __builtin_amdgcn_s_barrier();  // (0) K requested, max words cleared
    const uint32_t pre = nblk < (uint32_t)VRING ? nblk : (uint32_t)VRING;
    for (uint32_t bt = 0; bt < pre; ++bt) issue(bt);
    if (qkv.parts) {
      float x, x_unused;
      part_sums(vpl, x, x_unused);
      vnew = (uint16_t)f32_to_bf16_bits(x);
      if (pos_ok) qkv.v_cache[(bh * L + pos) * D + colbase + lane] = vnew;
      if (qkv.qkv_out) qkv.qkv_out[(uint64_t)row * 3 * HD + 2 * HD + (uint64_t)h * D + colbase + lane] = x;
    }
    lds_barrier();  // (1) scores, last NaN and first key written
    const uint32_t jn = *nan_word;
    if (jn != 0u && jn < len) lds_barrier();  // (1a) key after the last NaN
    __builtin_amdgcn_s_barrier();  // (2) exp~ written
    __builtin_amdgcn_s_barrier();  // (3) den written
    __builtin_amdgcn_s_barrier();  // (4) p written
    asm volatile("" ::: "memory");

    // Wait until at most `after` batches (8 loads each) are still in flight.
    auto wait_after = [&](uint32_t after) {
      switch (after) {
        case 0: FEW_WAIT_VMCNT(0); break;
        case 1: FEW_WAIT_VMCNT(8); break;
        case 2: FEW_WAIT_VMCNT(16); break;
        case 3: FEW_WAIT_VMCNT(24); break;
        default: FEW_WAIT_VMCNT(32); break;
      }
      asm volatile("" ::: "memory");
    };
    // Round b (after barrier (6) of b): the score waves make batch b + 1's
    // products while this wave adds batch b's.  Before that barrier this
    // wave has batch b + 1 in LDS (the batches issued after it, at most
    // VRING - 2 of them, may still be in flight) with the new value row in
    // place; after it, batch b's ring slot (its products are made) takes
    // batch b + VRING.  Lane = column colbase + lane: 16 reads of four
    // ascending products each, t ascending.
    const uint32_t pcol = kOffP + vw * HALF_PSLOT + (uint32_t)lane * 256u;
    const uint32_t pswz = (uint32_t)lane & 15u;
    float acc = __uint_as_float(0u);
    if (nblk > 0) {
      wait_after(nblk - 1 < (uint32_t)(VRING - 1) ? nblk - 1 : (uint32_t)(VRING - 1));
      put_new_val(0);
    }
    lds_barrier();  // (5) batch 0 in LDS
    for (uint32_t b = 0; b < nblk; ++b) {
      if (b + 1 < nblk) {
        wait_after(nblk - 2 - b < (uint32_t)(VRING - 2) ? nblk - 2 - b : (uint32_t)(VRING - 2));
        put_new_val(b + 1);
      }
      lds_barrier();  // (6) batch b's products written, batch b + 1 in LDS
      if (b + VRING < nblk) issue(b + VRING);
      uint32_t pbase = pcol + (b & 1u) * PSLOT_BYTES;
      asm volatile("" : "+v"(pbase));
      const lds_u8* pp = (const lds_u8*)smem + pbase;
      // four groups of four reads, each group added once it has landed
      // (at most 12 reads in flight: the LDS counter holds 15)
      f32x4_t pr[16];
      auto add4 = [&](int k0) {
#pragma unroll
        for (int k = k0; k < k0 + 4; ++k)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc = acc + pr[k][e];
      };
#pragma unroll
      for (uint32_t k = 0; k < 12; ++k) pr[k] = *(const lds_f32x4*)(pp + 16u * (k ^ pswz));
      FEW_WAIT_LGKM(8);
      add4(0);
#pragma unroll
      for (uint32_t k = 12; k < 16; ++k) pr[k] = *(const lds_f32x4*)(pp + 16u * (k ^ pswz));
      FEW_WAIT_LGKM(8);
      add4(4);
      FEW_WAIT_LGKM(4);
      add4(8);
      FEW_WAIT_LGKM(0);
      add4(12);
    }
    if (OUT_BF16)
      static_cast<uint16_t*>(o)[(uint64_t)qi * D + colbase + lane] = (uint16_t)f32_to_bf16_bits(acc);
    else
      static_cast<float*>(o)[(uint64_t)qi * D + colbase + lane] = acc;
    return;
  }

  // ------------------------------------------------------------ K waves
  // this wave's q, requested ahead of its K rows so it lands first (lane l:
  // elements 2l, 2l+1; partials mode: l and l + 64, the q / k parts' loads
  // first, then the K rows, then q / k added and rotated once the parts
  // are in -- the K requests do not wait for the parts)
  uint16_t q_lo = 0, q_hi = 0;
  uint32_t q_pair = 0;  // elements 2l, 2l+1 (unpacked after the K requests)
  uint16_t* kbuf = reinterpret_cast<uint16_t*>(smem + kOffKNew);  // the new key row, bf16
  const uint32_t blk_new = pos / 64u;  // the block holding the new row
  RopeLoads lq, lk;
  if (qkv.parts) {
    rope_loads(0, lq);
    // every score wave requests the new key's pair too (its loads go out
    // with q's); the wave whose blocks hold it uses it
    rope_loads(1, lk);
  } else {
    q_pair = *reinterpret_cast<const uint32_t*>(q + (uint64_t)qi * D + 2 * lane);
  }
  const int lrow = lane >> 2, lchunk = lane & 3;
  auto gload = [&](uint32_t blk, u32x4_t r[16]) {
#pragma unroll
    for (int seg = 0; seg < 4; ++seg)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t t = blk * 64 + lrow + 16 * i;
        if (t >= len) t = 0;  // in bounds; such a score is never read
        r[4 * seg + i] = *reinterpret_cast<const u32x4_t*>(kb + (uint64_t)t * D + seg * 32 + lchunk * 8);
      }
  };
  // (loads are unconditional: rows past len read row 0, so no copies of
  // the register blocks are needed to merge loaded and not-loaded paths)
  u32x4_t ra[16], rb[16];
  const uint32_t b0 = (uint32_t)wave;
  gload(b0, ra);
  gload(b0 + KWAVES, rb);
  if (qkv.parts) {
    float x1, x2, y1, y2, kx1, kx2, ky1, ky2;
    rope_pair(lq, x1, x2, y1, y2);
    rope_pair(lk, kx1, kx2, ky1, ky2);
    q_lo = (uint16_t)f32_to_bf16_bits(y1);
    q_hi = (uint16_t)f32_to_bf16_bits(y2);
    if (wave == 0) {
      uint16_t* dq = qkv.q_out + (uint64_t)row * HD + (uint64_t)h * D;
      dq[lane] = q_lo;
      dq[lane + 64] = q_hi;
      if (qkv.qkv_out) {
        float* dx = qkv.qkv_out + (uint64_t)row * 3 * HD + (uint64_t)h * D;
        dx[lane] = x1;
        dx[lane + 64] = x2;
      }
    }
    if (wave == (int)(blk_new % KWAVES)) {
      // the new key: into this wave's LDS row buffer, and to the cache
      const uint16_t k1 = (uint16_t)f32_to_bf16_bits(ky1), k2 = (uint16_t)f32_to_bf16_bits(ky2);
      kbuf[lane] = k1;
      kbuf[lane + 64] = k2;
      if (pos_ok) {
        uint16_t* dk = qkv.k_cache + (bh * L + pos) * D;
        dk[lane] = k1;
        dk[lane + 64] = k2;
      }
      if (qkv.qkv_out) {
        float* dx = qkv.qkv_out + (uint64_t)row * 3 * HD + HD + (uint64_t)h * D;
        dx[lane] = kx1;
        dx[lane + 64] = kx2;
      }
    }
  }
  unsigned char* st = smem + kOffK + wave * KSTAGE_WAVE;
  float* qf = reinterpret_cast<float*>(smem + wave * 512);
  // one block: its 64 scores into sp, its max-fold state into the block
  // state arrays
  auto fold = [&](uint32_t blk, const u32x4_t r[16]) {
    float acc = __uint_as_float(0u);
#pragma unroll
    for (int seg = 0; seg < 4; ++seg) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<u32x4_t*>(st + (lrow + 16 * i) * KSTAGE_ROW + kswz(lrow, lchunk)) = r[4 * seg + i];
      wave_sync();
      const unsigned char* myrow = st + lane * KSTAGE_ROW;
#pragma unroll
      for (int ch = 0; ch < 4; ++ch) {
        const u32x4_t kv = *reinterpret_cast<const u32x4_t*>(myrow + kswz(lane, ch));
        const f32x4_t q0 = *reinterpret_cast<const f32x4_t*>(qf + seg * 32 + ch * 8);
        const f32x4_t q1 = *reinterpret_cast<const f32x4_t*>(qf + seg * 32 + ch * 8 + 4);
        float p;
        p = q0[0] * bf16lo(kv[0]); acc = acc + p;
        p = q0[1] * bf16hi(kv[0]); acc = acc + p;
        p = q0[2] * bf16lo(kv[1]); acc = acc + p;
        p = q0[3] * bf16hi(kv[1]); acc = acc + p;
        p = q1[0] * bf16lo(kv[2]); acc = acc + p;
        p = q1[1] * bf16hi(kv[2]); acc = acc + p;
        p = q1[2] * bf16lo(kv[3]); acc = acc + p;
        p = q1[3] * bf16hi(kv[3]); acc = acc + p;
      }
      wave_sync();  // the slice is rewritten by the next segment
    }
    // stored unconditionally (sp holds whole blocks; entries past len are
    // never read), so the dot product stays where its operands arrive
    // instead of sinking into a branch that keeps them all live
    const uint32_t t = blk * 64 + (uint32_t)lane;
    const float sv = acc * scale;
    sp[t] = sv;
    if (t + 1 == len) *last_slot = sv;  // read by every score wave below
    // one LDS atomic per wave and block: the block's last NaN, and the key
    // of its first maximal score (the wave's largest monotone bits, then
    // the lowest lane holding them)
    const bool in = t < len, nan = sv != sv;
    const uint64_t nans = __builtin_amdgcn_ballot_w64(in && nan);
    if (nans != 0u && lane == 0)
      __hip_atomic_fetch_max(nan_word, blk * 64 + (63u - (uint32_t)__builtin_clzll(nans)) + 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
    const uint32_t bits = __float_as_uint(sv);
    const uint32_t mono = (in && !nan) ? mono_bits(bits) : 0u;
    const uint32_t m = wave_umax(mono);
    if (m != 0u) {
      const uint32_t wl = (uint32_t)__builtin_ctzll(__builtin_amdgcn_ballot_w64(mono == m));
      const uint32_t wbits = (uint32_t)__builtin_amdgcn_readlane((int)bits, (int)wl);
      if (lane == 0)
        __hip_atomic_fetch_max(&key_word[0], make_key(m, blk * 64 + wl, wbits), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  if (wave == 0 && lane == 0) {
    *nan_word = 0u;
    key_word[0] = 0u;
    key_word[1] = 0u;
  }
  lds_barrier();  // (0) K requested (V follows it), max words cleared
  if (qkv.parts) {
    qf[lane] = bf16_to_f32(q_lo);
    qf[lane + 64] = bf16_to_f32(q_hi);
  } else {
    qf[2 * lane] = bf16lo(q_pair);
    qf[2 * lane + 1] = bf16hi(q_pair);
  }
  wave_sync();
  // partials mode: the rows of block blk_new in registers r, row pos % 64
  // replaced by the new key (row lrow + 16 i of segment seg is r[4 seg + i])
  auto put_new_key = [&](u32x4_t r[16]) {
    const uint32_t rp = pos & 63u;
    const bool mine = (uint32_t)lrow == (rp & 15u);
#pragma unroll
    for (int seg = 0; seg < 4; ++seg) {
      const u32x4_t nv = *reinterpret_cast<const u32x4_t*>(kbuf + seg * 32 + lchunk * 8);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (mine && (uint32_t)i == (rp >> 4)) r[4 * seg + i] = nv;
    }
  };
  const bool new_key = qkv.parts && pos_ok;  // then len = pos + 1 >= 1
  for (uint32_t bk = b0; bk < nblk; bk += 2 * KWAVES) {
    if (new_key && bk == blk_new) put_new_key(ra);
    fold(bk, ra);
    gload(bk + 2 * KWAVES, ra);
    if (bk + KWAVES < nblk) {
      if (new_key && bk + KWAVES == blk_new) put_new_key(rb);
      fold(bk + KWAVES, rb);
    }
    gload(bk + 3 * KWAVES, rb);
  }
  lds_barrier();  // (1) scores, last NaN and first key written
  const uint32_t stride = 64u * KWAVES;
  const uint32_t jn = *nan_word;  // last NaN position + 1, 0 if none
  uint64_t key = key_word[0];
  if (jn != 0u && jn < len) {
    // the first maximum of the scores after the last NaN
    for (uint32_t t = jn + (uint32_t)(wave * 64 + lane); t < len; t += stride)
      __hip_atomic_fetch_max(&key_word[1], max_key(sp[t], t), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    lds_barrier();  // (1a)
    key = key_word[1];
  }
  float mx;
  if (jn != 0u && jn == len)
    mx = *last_slot;  // the final score is NaN: the fold returns it
  else
    mx = key == 0u ? __uint_as_float(0xFF800000u) : key_score(key);
  for (uint32_t t = (uint32_t)(wave * 64 + lane); t < len; t += stride) sp[t] = exp_approx(sp[t] - mx);
  lds_barrier();  // (2) exp~ written
  if (wave == 0) {
    // the one sequential fold den = (((0 + e_0) + e_1) + ...) in ascending t
    const float den = serial_sum_wave_long(sp, len);
    if (lane == 0) *den_slot = den;
  }
  lds_barrier();  // (3) den written
  const float den = *den_slot;
  for (uint32_t t = (uint32_t)(wave * 64 + lane); t < len; t += stride) sp[t] = sp[t] / den;
  lds_barrier();  // (4) p written

  // Products p_t * v_{t,c} (one rounded multiply each) of batch b into
  // product slot b % 2, in the order the V waves add them: column c of
  // half h (of the workgroup's halves) at kOffP + (b % 2) PSLOT_BYTES +
  // h HALF_PSLOT + 256 c, its 16-byte chunk t / 4 at chunk index
  // (t / 4) ^ (c % 16).  A batch is 16 units of 8 rows x 64 columns (unit
  // u: half u / 8, rows 8 (u % 8) ..; the split form: 8 units of its one
  // half), wave w making units w, w + 6, w + 12.  Per unit: two transposing reads
  // (lane 16g + i receives column 16g + i of rows 4j .. 4j + 3), p of the 8
  // rows by a DPP row broadcast, one 16-byte write per four rows.  In the
  // last, partial batch rows past len (they hold row 0 and sp holds no p for
  // them) get +0, which the V waves' sums absorb unchanged (they start at +0
  // and an add never turns them into -0).
  const uint32_t tr_off = (4u * (((uint32_t)lane & 15u) >> 2)) * 32u +
                          2u * (16u * ((uint32_t)lane >> 4) + 4u * ((uint32_t)lane & 3u));
  const uint32_t nunits = SPLIT ? (wave < 2 ? 2u : 1u) : (wave < 4 ? 3u : 2u);
  auto produce = [&](uint32_t b) {
    i16x4_t v4[3][2];
    float p8[3];
#pragma unroll
    for (uint32_t rep = 0; rep < 3; ++rep) {
      if (rep < nunits) {
        const uint32_t unit = (uint32_t)wave + 6u * rep, half = SPLIT ? 0u : unit >> 3, o8 = unit & 7u;
        uint32_t vbase = kOffV + half * (VRING * VB_BYTES) + (b % VRING) * VB_BYTES + o8 * 8u * 128u + tr_off;
        uint32_t pbase = kOffState + (b * 64u + o8 * 8u + ((uint32_t)lane & 7u)) * 4u;
        asm volatile("" : "+v"(vbase), "+v"(pbase));
        p8[rep] = *(const __attribute__((address_space(3))) float*)((const lds_u8*)smem + pbase);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          v4[rep][j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)((const lds_u8*)smem + vbase + 512 * j));
      }
    }
    const bool partial = (b + 1u) * 64u > len;
#pragma unroll
    for (uint32_t rep = 0; rep < 3; ++rep) {
      if (rep < nunits) {
        const uint32_t unit = (uint32_t)wave + 6u * rep, half = SPLIT ? 0u : unit >> 3, o8 = unit & 7u;
        const uint32_t t0 = b * 64u + o8 * 8u;
        uint32_t wbase = kOffP + (b & 1u) * PSLOT_BYTES + half * HALF_PSLOT + (uint32_t)lane * 256u;
        asm volatile("" : "+v"(wbase));
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          f32x4_t pr;
#pragma unroll
          for (int e = 0; e < 4; ++e) pr[e] = row_bcast(p8[rep], 4 * j + e) * bf16_to_f32((uint16_t)v4[rep][j][e]);
          if (partial) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (t0 + (uint32_t)(4 * j + e) >= len) pr[e] = __uint_as_float(0u);
          }
          *(lds_f32x4*)((lds_u8*)smem + wbase + 16u * ((2u * o8 + (uint32_t)j) ^ ((uint32_t)lane & 15u))) = pr;
        }
      }
    }
  };
  lds_barrier();  // (5) batch 0 in LDS
  if (nblk > 0) produce(0);
  for (uint32_t b = 0; b < nblk; ++b) {
    lds_barrier();  // (6) batch b's products written, batch b + 1 in LDS
    if (b + 1 < nblk) produce(b + 1);
  }
}

}  // namespace

extern "C" __global__ __launch_bounds__(512) void catena_attn_few_bf16_d128_f32out(
    const uint16_t* __restrict__ q, const uint16_t* k, const uint16_t* v, const uint32_t* __restrict__ lens,
    float* __restrict__ o, uint32_t H, uint32_t L, uint32_t Tq, float scale, FewQkv qkv) {
  attn_few_body<false, false>(q, k, v, lens, o, H, L, Tq, scale, qkv);
}

extern "C" __global__ __launch_bounds__(512) void catena_attn_few_bf16_d128_bf16out(
    const uint16_t* __restrict__ q, const uint16_t* k, const uint16_t* v, const uint32_t* __restrict__ lens,
    uint16_t* __restrict__ o, uint32_t H, uint32_t L, uint32_t Tq, float scale, FewQkv qkv) {
  attn_few_body<true, false>(q, k, v, lens, o, H, L, Tq, scale, qkv);
}

// the split form: grid = 2 x pairs, block = 448 (7 waves)
extern "C" __global__ __launch_bounds__(448) void catena_attn_few_split_bf16_d128_f32out(
    const uint16_t* __restrict__ q, const uint16_t* k, const uint16_t* v, const uint32_t* __restrict__ lens,
    float* __restrict__ o, uint32_t H, uint32_t L, uint32_t Tq, float scale, FewQkv qkv) {
  attn_few_body<false, true>(q, k, v, lens, o, H, L, Tq, scale, qkv);
}

extern "C" __global__ __launch_bounds__(448) void catena_attn_few_split_bf16_d128_bf16out(
    const uint16_t* __restrict__ q, const uint16_t* k, const uint16_t* v, const uint32_t* __restrict__ lens,
    uint16_t* __restrict__ o, uint32_t H, uint32_t L, uint32_t Tq, float scale, FewQkv qkv) {
  attn_few_body<true, true>(q, k, v, lens, o, H, L, Tq, scale, qkv);
}
