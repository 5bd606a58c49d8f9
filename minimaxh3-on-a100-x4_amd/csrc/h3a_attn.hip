// Dense and block-sparse non-causal flash-attention forward for gfx950 (MI355X),
// head_dim 128, bf16 in/out, fp32 accumulation.
//
// What it computes follows the reference kernel fa3_sm80_h3_kernel
// (attn_sm80/fa3_sm80_h3.cu:252-458): scale and mask keys >= Skv to -inf
// (:355-365), online softmax with running max/sum (:367-401), P rounded to
// bf16 before the PV product while the row sum uses unrounded p (:386-394,
// :405-420), O = acc / l with row-guarded stores (:443-457).  How it is
// computed is CDNA4-specific:
//
//  * Each wave keeps 32 query rows as the B operand of
//    v_mfma_f32_32x32x16_bf16 in VGPRs and produces the score tile
//    transposed, S^T = K Q^T, so every lane owns a single query row (column
//    l%32) and 32 of the 64 keys of a stage.  That layout is already the B
//    operand of O^T += V^T P^T: P goes from the score accumulators straight
//    into the PV MFMA (no LDS round trip).  V stays row-major in LDS and its A
//    operand is read with ds_read_b64_tr_b16 (LDS transpose reads), addressed
//    so that the key order matches the score accumulator's.
//  * Dense (attn_fwd_pingpong_kernel): 8 waves = 256 query rows per
//    workgroup, in two groups with one wave of each per SIMD.  Every 64-key
//    stage is a matrix-core cluster and a softmax cluster separated by
//    workgroup barriers, group B one cluster behind group A, so one wave per
//    SIMD issues MFMAs while the other issues the softmax's VALU work.  K/V
//    stages are double-buffered in LDS (256-byte rows, XOR-swizzled at
//    16-byte granularity for conflict-free operand reads) and fetched by LDS
//    DMA (buffer_load_dwordx4 ... lds) from group B.  The softmax runs against
//    a stale reference max and takes a row max only when a stage's p sum
//    overflows its bound.  A split tail cuts the last, partly filled round of
//    query tiles into key ranges merged by split_combine_kernel.
//  * Block-sparse (attn_fwd_pingpong_kernel with kSparse): the ping-pong
//    over a pair of query blocks, one per group, each with its own LUT row
//    and K/V stream fetched by LDS DMA into swizzled rows; a group issues its
//    K fetch at the top of its softmax slot (while the other group's MFMAs
//    run) and its V fetch right after its matrix cluster.  LUT entries are
//    read ahead.  128-row blocks: each wave takes 32 rows against all 64 keys
//    of a stage.  64-row blocks (kKeySplit): a group's 4 waves are 2 query
//    slices x 2 key halves, merged at the end.
//  * Every stage's buffer resource is rebased on its first key and covers only
//    the valid rows, so rows past Skv arrive as zeros and offsets stay
//    loop-invariant; exp2-based softmax with scale*log2(e) folded into one
//    FMA; workgroup ids are remapped XCD-aware (xcd_remap).
#include <atomic>
#include <climits>
#include <type_traits>

#include "h3a_device.h"
#include "h3a_internal.h"
#include "h3a_lut.h"
#include "h3a_queue.h"
#include "h3a_stale.h"

namespace h3a {

// Phase profile build (libh3attn_prof.so): the ping-pong kernel stamps the
// shader clock at its cluster boundaries (see PhaseClock).
#ifndef H3A_PROFILE
#define H3A_PROFILE 0
#endif

constexpr int kD = 128;
constexpr int kBN = 64;               // keys per pipeline stage
constexpr float kRescaleSlack = 8.f;  // log2 headroom before the running max is refreshed

__device__ __forceinline__ int stage_key0(const AttnArgs &a, int t, int kb) {
  return lut_stage_key0(t, kb, a.nkb, a.blk_k, a.sub, a.Skv);
}

// ---------------------------------------------------------------------------
// LDS layout of a 64-key K or V stage: the row pitch, which 16-byte global
// chunk each 16-byte LDS slot holds, and how the MFMA operand reads address
// the stage.  Bank-conflict free for the reads below (SQ_LDS_BANK_CONFLICT = 0
// measured).  The kernels take the layout as a template parameter L.
//
// SwzLayout: 256-byte rows; chunk c of row r sits in slot c ^ swz(r).
//   K: swz(r) = r & 15.  A 128-bit read of one chunk by 16 consecutive rows
//      (the A operand of the score MFMA) hits 16 distinct bank groups.
//   V: swz(r) = 4 * (r & 3).  A transpose read by 32 lanes covers 4 rows x
//      4 chunks, which land on 16 distinct bank groups: all 64 banks once.
//   Read offsets are base ^ const, held per lane.
struct SwzLayout {
  static constexpr int kKRow = 256, kVRow = 256;  // bytes
  static constexpr int kKSlots = 16, kVSlots = 16;
  __device__ __forceinline__ static int k_chunk(int r, int slot) { return slot ^ (r & 15); }
  __device__ __forceinline__ static int v_chunk(int r, int slot) { return slot ^ (4 * (r & 3)); }
  // Lane's A-operand chunk of k-step 0 (row l32, chunk g); k-step ks reads
  // chunk 2*ks + g, i.e. offset k_base ^ (32*ks).
  __device__ __forceinline__ static int k_base(int l32, int g) {
    return l32 * kKRow + 32 * ((l32 >> 1) & 7) + 16 * (g ^ (l32 & 1));
  }
  __device__ __forceinline__ static int k_off(int kb, int ks) { return kb ^ (32 * ks); }
  // Column block dt of the transpose reads is chunk 4*dt + c of the row,
  // stored in slot (4*dt + c) ^ 4*(row & 3): offset v_base ^ (64*dt).
  __device__ __forceinline__ static int v_base(int lane) {
    const int i = (lane & 15) >> 2;
    const int row = 4 * (lane >> 5) + i;
    const int c = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    return row * kVRow + 64 * i + 16 * c + 8 * (lane & 1);
  }
  __device__ __forceinline__ static int v_off(int vb, int dt) { return vb ^ (64 * dt); }
};

template <class L, int ROWS = kBN>
struct StageBytes {
  static constexpr int kK = ROWS * L::kKRow;
  static constexpr int kV = ROWS * L::kVRow;
};

// Global -> LDS staging of one ROWS-key K or V stage by LDS DMA.  Instruction
// t fills the 64 consecutive 16-byte slots 64t..64t+63 of the stage (1 KiB);
// each lane fetches the global chunk that its slot holds under the layout.
// The NW waves of the stream issue instructions t = wave, wave+NW, ...  The
// buffer resource is rebased on the stage's first key and covers exactly its
// valid rows, so rows >= Skv arrive as zeros (masked keys never carry
// NaN/Inf) and the per-lane offsets are loop-invariant.
template <int NW, class L, bool kIsV, int ROWS = kBN>
struct TileDma {
  static constexpr int kWaves = NW;
  static constexpr int kSlots = kIsV ? L::kVSlots : L::kKSlots;  // per row
  static constexpr int kInstTotal = ROWS * kSlots / 64;           // 64 lanes per instruction
  static constexpr int kInst = (kInstTotal + NW - 1) / NW;        // per wave (the last may be idle)
  static_assert(ROWS * kSlots % 64 == 0, "a stage is a whole number of DMA instructions");
  // With 16-slot rows and NW a multiple of 4, instruction i covers rows
  // 4*(wave + i*NW) + lane/16: the swizzle (row & 15 or row & 3) does not
  // depend on i, so the offsets are off[0] + i * 4*NW rows and one register
  // holds them all.
  static constexpr bool kAffine = kSlots == 16 && NW % 4 == 0;
  uint32_t off[kAffine ? 1 : kInst];
  uint32_t step;  // bytes between instructions when kAffine (wave-uniform)
  int wave;       // wave-uniform

  __device__ __forceinline__ void init(int64_t ss, int wave_uniform, int lane) {
    wave = wave_uniform;
    step = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(4 * NW * ss * 2));
#pragma unroll
    for (int i = 0; i < (kAffine ? 1 : kInst); ++i) {
      const int slot = 64 * (wave + i * NW) + lane;
      const int row = slot / kSlots, sl = slot % kSlots;
      const int chunk = kIsV ? L::v_chunk(row, sl) : L::k_chunk(row, sl);
      off[i] = (uint32_t)(((int64_t)(row < ROWS ? row : ROWS - 1) * ss + chunk * 8) * 2);
    }
  }
  // Offsets of instructions 0, 1, ... in issue order: `cur` starts at
  // first() and next() moves it on.  The add is opaque to the compiler, which
  // would otherwise hoist all kInst offsets out of the stage loop and keep
  // them in registers.  Without kAffine the cursor is the byte offset added
  // to every instruction's own offset (the stage's, for a descriptor of the
  // whole (b,h) slice).
  __device__ __forceinline__ uint32_t first() const { return kAffine ? off[0] : 0u; }
  __device__ __forceinline__ uint32_t next(uint32_t cur) const {
    if constexpr (kAffine) {
      uint32_t r;
      asm volatile("v_add_u32 %0, %1, %2" : "=v"(r) : "v"(cur), "s"(step));
      return r;
    } else {
      return cur;
    }
  }
  // Buffer descriptor of the stage that starts at key0 (valid rows only).
  __device__ __forceinline__ u32x4 desc(const uint16_t *base, int64_t ss, int key0, int Skv) const {
    const int rows = Skv - key0 >= ROWS ? ROWS : (Skv > key0 ? Skv - key0 : 0);
    return stage_desc(stage_ptr(base, key0, ss), ss, rows);
  }
  // Instruction i (0 <= i < kInst, a compile-time index) of this wave's
  // share; `cur` is its offset cursor (first(), then next() once per
  // instruction) and m0 the LDS address of its 1 KiB: that of instruction
  // 0, lds_address(tile) + 1024 * wave, plus 1024 * NW per instruction,
  // advanced by opaque_sadd so that the compiler does not keep every
  // instruction's address of both buffers live in SGPRs.
  __device__ __forceinline__ void issue_one(u32x4 d, int i, uint32_t cur, uint32_t m0) const {
    if (kInstTotal % NW == 0 || wave + i * NW < kInstTotal)
      buffer_load_lds_b128(d, kAffine ? cur : off[i] + cur, m0);
  }
  __device__ __forceinline__ void issue(const uint16_t *base, int64_t ss, int key0, int Skv,
                                        uint16_t *tile) const {
    issue_range<0, kInst>(base, ss, key0, Skv, tile);
  }
  // Instructions I0 .. I1-1 of this wave's share.
  template <int I0, int I1>
  __device__ __forceinline__ void issue_range(const uint16_t *base, int64_t ss, int key0, int Skv,
                                              uint16_t *tile) const {
    if constexpr (I1 > I0) issue_desc<I0, I1>(desc(base, ss, key0, Skv), tile);
  }
  // The same with the stage's descriptor given (StageCursor::desc).
  template <int I0, int I1>
  __device__ __forceinline__ void issue_desc(u32x4 d, uint16_t *tile) const {
    issue_desc_off<I0, I1>(d, tile, 0u);
  }
  // The same with a descriptor of the whole (b,h) slice and the stage's byte
  // offset in it, soff, added to every lane's offset (one v_add).
  template <int I0, int I1>
  __device__ __forceinline__ void issue_desc_off(u32x4 d, uint16_t *tile, uint32_t soff) const {
    if constexpr (I1 > I0) {
      uint32_t cur = first() + soff;
#pragma unroll
      for (int i = 0; i < I0; ++i) cur = next(cur);
      uint32_t m0 = lds_address(tile) + (uint32_t)(wave + I0 * NW) * 1024u;
#pragma unroll
      for (int i = I0; i < I1; ++i) {
        issue_one(d, i, cur, m0);
        if (i + 1 < I1) {
          cur = next(cur);
          m0 = opaque_sadd<1024u * NW>(m0);
        }
      }
    }
  }
  // Common staging interface: start() at the top of a stage, finish() at its
  // end; kAsync stagers need a vmcnt wait before the stage's barrier.
  static constexpr bool kAsync = true;
  __device__ __forceinline__ void start(const uint16_t *base, int64_t ss, int key0, int Skv,
                                        uint16_t *tile) {
    issue(base, ss, key0, Skv, tile);
  }
  __device__ __forceinline__ void finish(uint16_t *) const {}
};

// One wave's share of a stage's TileDma fetch issued one instruction at a
// time (issue_desc taken apart), to spread it over a matrix cluster.
template <class Dma>
struct DmaSeq {
  static constexpr int kCount = Dma::kInst;
  const Dma &dma;
  u32x4 d;
  uint32_t cur, m0;
  int i;
  // soff: the stage's byte offset when d describes the whole (b,h) slice.
  __device__ __forceinline__ DmaSeq(const Dma &dma_, u32x4 d_, uint16_t *tile, uint32_t soff)
      : dma(dma_), d(d_), cur(dma_.first() + soff), m0(lds_address(tile) + (uint32_t)dma_.wave * 1024u), i(0) {}
  __device__ __forceinline__ void issue() {
    dma.issue_one(d, i, cur, m0);
    ++i;
    if (i < Dma::kInst) {
      cur = dma.next(cur);
      m0 = opaque_sadd<1024u * Dma::kWaves>(m0);
    }
  }
};

// Wave-uniform position of a K or V stream in a contiguous range of key
// stages: the byte address of the next stage's first row and the number of
// valid rows from there on (it goes negative past the range's end, where the
// descriptor covers nothing and the DMA writes zeros).  advance() moves on by
// one stage with one opaque 64-bit scalar add; rebuilding the address as
// base + key0 * stride every stage costs a 64-bit multiply chain on the
// scalar unit in the middle of the issuing wave's DMA burst.
template <int ROWS>
struct StageCursor {
  uint32_t lo, hi, step_lo, step_hi, ss2;
  int rows_left;
  __device__ __forceinline__ void init(const uint16_t *base, int64_t ss, int key0, int key_end) {
    const uint64_t addr = reinterpret_cast<uint64_t>(base) + (uint64_t)((int64_t)key0 * ss * 2);
    const uint64_t step = (uint64_t)((int64_t)ROWS * ss * 2);
    lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)addr);
    hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(addr >> 32));
    step_lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)step);
    step_hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(step >> 32));
    ss2 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(ss * 2));
    rows_left = __builtin_amdgcn_readfirstlane(key_end - key0);
  }
  // The V# of the current stage, as stage_desc builds it: valid rows only.
  __device__ __forceinline__ u32x4 desc() const {
    const int rows = rows_left >= ROWS ? ROWS : (rows_left > 0 ? rows_left : 0);
    const uint32_t bytes = rows > 0 ? (uint32_t)(rows - 1) * ss2 + 256u : 0u;
    return u32x4{lo, hi & 0xffffu, bytes, (uint32_t)kBufferConfig};
  }
  __device__ __forceinline__ void advance() {
    asm volatile("s_add_u32 %0, %0, %2\n\ts_addc_u32 %1, %1, %3"
                 : "+s"(lo), "+s"(hi)
                 : "s"(step_lo), "s"(step_hi)
                 : "scc");
    rows_left -= ROWS;
  }
};

// A stage's scores live in NSUB accumulators of 32 keys: s[u] holds keys
// 32u..32u+31 of the stage.  In the S^T accumulator layout lane l owns query
// l%32; register r of s[u] holds key 32u + 8*(r/4) + 4*(l/32) + r%4.

// score_tile calls hook(k-step) after each k-step's MFMAs and pv_tile
// hook(4 * key step + dim tile) after each MFMA (by default nothing): where a
// matrix cluster's LDS DMA instructions go when they are spread over it.
struct NoHook {
  __device__ __forceinline__ void operator()(int) const {}
};

// S^T (32*NSUB keys x 32 queries of this wave) = K_stage Q^T.
template <class L, int NSUB, class Hook = NoHook>
__device__ __forceinline__ void score_tile(const uint16_t *kbuf, const u32x4 (&qf)[8], int k_rd,
                                           f32x16 (&s)[NSUB], Hook hook = Hook{}) {
#pragma unroll
  for (int u = 0; u < NSUB; ++u) s[u] = f32x16{0.f};
  const char *kb = reinterpret_cast<const char *>(kbuf);
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const char *p = kb + L::k_off(k_rd, ks);
#pragma unroll
    for (int u = 0; u < NSUB; ++u) {
      const u32x4 a = *(const u32x4 *)(p + 32 * u * L::kKRow);
      s[u] = mfma_32x32x16(a, qf[ks], s[u]);
    }
    hook(ks);
  }
}

// P^T fragments for the 2*NSUB sixteen-key steps, straight from the S^T
// registers.  Step ks, k-slot (g = lane/32, e) carries key
// 16*ks + 8*(e/4) + 4*g + e%4.
template <int NSUB>
__device__ __forceinline__ void pack_p(const f32x16 (&s)[NSUB], u32x4 (&pf)[2 * NSUB]) {
#pragma unroll
  for (int u = 0; u < NSUB; ++u)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      pf[2 * u + h] = u32x4{pack_bf16x2(s[u][8 * h + 0], s[u][8 * h + 1]),
                            pack_bf16x2(s[u][8 * h + 2], s[u][8 * h + 3]),
                            pack_bf16x2(s[u][8 * h + 4], s[u][8 * h + 5]),
                            pack_bf16x2(s[u][8 * h + 6], s[u][8 * h + 7])};
}

// V transpose reads.  Within each 16-lane group a ds_read_b64_tr_b16 gives
// lane j element j%4 of the 4 consecutive bf16 that lanes 4k + j/4 address
// (k = 0..3).  Lane i of group t points at row 4*(t/2) + i/4 (+16*ks, +8 for
// k-slots 4..7) and columns 16*(t%2) + 4*(i%4) (+32*dt), so lane l receives
// V[key][32*dt + l%32] for the 4 keys of its k-slots, in the score
// accumulator's key order.  L::v_base / L::v_off place that in the layout.
// O^T (128 dims x 32 queries) += V^T_stage P^T over NKS sixteen-key steps.
template <class L, int NKS, class Hook = NoHook>
__device__ __forceinline__ void pv_tile(const uint16_t *vbuf, const u32x4 (&pf)[NKS], int v_rd,
                                        f32x16 (&o)[4], Hook hook = Hook{}) {
  const char *vb = reinterpret_cast<const char *>(vbuf);
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const char *p = vb + L::v_off(v_rd, dt) + 16 * ks * L::kVRow;
      const u32x2 lo = lds_read_tr16_b64(reinterpret_cast<const uint16_t *>(p));
      const u32x2 hi = lds_read_tr16_b64(reinterpret_cast<const uint16_t *>(p + 8 * L::kVRow));
      o[dt] = mfma_32x32x16(u32x4{lo.x, lo.y, hi.x, hi.y}, pf[ks], o[dt]);
      hook(4 * ks + dt);
    }
  }
}

// Max of N values as a tree of v_max3 (depth log3 N), not a dependent chain:
// the softmax cluster is latency-bound.
template <int N>
__device__ __forceinline__ float max_tree(const float (&v)[N]) {
  if constexpr (N == 1) {
    return v[0];
  } else if constexpr (N == 2) {
    return fmaxf(v[0], v[1]);
  } else {
    constexpr int M = (N + 2) / 3;
    float t[M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
      if (3 * i + 2 < N)
        t[i] = fmaxf(fmaxf(v[3 * i], v[3 * i + 1]), v[3 * i + 2]);
      else if (3 * i + 1 < N)
        t[i] = fmaxf(v[3 * i], v[3 * i + 1]);
      else
        t[i] = v[3 * i];
    }
    return max_tree<M>(t);
  }
}

// Row max of a masked score stage (all sub-tiles, both lane halves), in
// scale*log2(e) units.
template <int NSUB>
__device__ __forceinline__ float tile_max(const f32x16 (&s)[NSUB], float sl2) {
  float v[16 * NSUB];
#pragma unroll
  for (int u = 0; u < NSUB; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) v[16 * u + r] = s[u][r];
  return half_swap_max(max_tree<16 * NSUB>(v)) * sl2;
}

// This lane's share of the row sum of a stage's p values (a tree of adds).
template <int NSUB>
__device__ __forceinline__ float tile_sum(const f32x16 (&s)[NSUB]) {
  float a[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    a[r] = s[0][r];
    if constexpr (NSUB >= 2) a[r] += s[1][r];
    if constexpr (NSUB == 4) a[r] += s[2][r] + s[3][r];
  }
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
    for (int r = 0; r < w; ++r) a[r] += a[r + w];
  return a[0];
}

// Keys >= Skv of the stage starting at key0 -> -inf (tail stage only).
template <int NSUB>
__device__ __forceinline__ void mask_tail(f32x16 (&s)[NSUB], int key0, int Skv, int g) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int kk = key0 + 8 * (r >> 2) + 4 * g + (r & 3);
#pragma unroll
    for (int u = 0; u < NSUB; ++u)
      if (kk + 32 * u >= Skv) s[u][r] = kNegInf;
  }
}

// Tile-mask sparse attention (64-row key-split pairs over 32-key columns,
// each with an 8-bit mask of kept 16x16 sub-blocks): the scores of this
// wave's column whose sub-block bit is clear -> -inf.  Bit 2*i + j covers
// rows 16i..16i+15 of the 64-row query block and keys 16j..16j+15 of the
// column.  The lane's query row is 32*rq + l32; its scores s[0][r] are keys
// 8*(r/4) + 4*g + r%4 of the column, so registers 0-7 lie in key sub-block 0
// and registers 8-15 in 1.
template <int NSUB>
__device__ __forceinline__ void apply_tile_mask(f32x16 (&s)[NSUB], uint32_t mask, int rq, int l32) {
  static_assert(NSUB == 1, "tile masks apply to the 32-key waves of the key-split kernel");
  const uint32_t bits = mask >> (2 * (2 * rq + (l32 >> 4)));
  const bool k0 = (bits & 1u) != 0, k1 = (bits & 2u) != 0;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    s[0][r] = k0 ? s[0][r] : kNegInf;
    s[0][r + 8] = k1 ? s[0][r + 8] : kNegInf;
  }
}

// ---------------------------------------------------------------------------
// Softmax of one score stage (32*NSUB keys), in place: S -> P (bf16 pairs in
// pf), the running max m and this lane's share of the row sum of the
// unrounded p.  m is refreshed lazily: only when some row of the wave exceeds
// it by more than kRescaleSlack (p then stays <= 2^kRescaleSlack), and O and l
// are rescaled only then.  VALU work only.
template <int NSUB>
__device__ __forceinline__ void softmax_stage(f32x16 (&s)[NSUB], int key0, int Skv, int g, float sl2,
                                              float &m, float &lsum, f32x16 (&o)[4],
                                              u32x4 (&pf)[2 * NSUB]) {
  if (key0 + 32 * NSUB > Skv) mask_tail<NSUB>(s, key0, Skv, g);
  const float mx = tile_max<NSUB>(s, sl2);
  if (__builtin_amdgcn_ballot_w64(mx > m + kRescaleSlack) != 0) {
    const float mnew = fmaxf(m, mx);
    const float alpha = fast_exp2(m - ((mnew == kNegInf) ? 0.f : mnew));
    m = mnew;
    lsum *= alpha;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
  }
  const float muse = (m == kNegInf) ? 0.f : m;
#pragma unroll
  for (int u = 0; u < NSUB; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[u][r] = fast_exp2(fmaf(s[u][r], sl2, -muse));
  pack_p<NSUB>(s, pf);
  lsum += tile_sum<NSUB>(s);
}

// Softmax of one score stage against the running reference m without
// computing the stage's row max.  p = 2^(s*sl2 - m) is formed, packed and
// summed straight away; only if some lane's stage sum exceeds kStaleSumLimit
// or is not finite (stage_sum_needs_refresh; +inf when a score ran 128 or
// more above m) does the wave take the row max, refresh m, rescale O and l
// and redo the stage.  m must be finite on entry (the first stage of a key
// range uses softmax_stage, which sets m to that stage's row max, so every
// later row sum is >= 1).  Every accepted p is then <= its stage sum <=
// 2^16 instead of <= 1: bf16 rounding of P and the fp32 sums are relative,
// so the normalised O is unchanged, and the bound on O that this leaves is
// given with kStaleSumLimit.
template <int NSUB>
__device__ __forceinline__ void exp_pack_sum(const f32x16 (&s)[NSUB], float sl2, float m,
                                             u32x4 (&pf)[2 * NSUB], float &ps) {
  float a[16];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int r = 8 * h + 2 * w;
      float p0[NSUB], p1[NSUB];
#pragma unroll
      for (int u = 0; u < NSUB; ++u) {
        p0[u] = fast_exp2(fmaf(s[u][r], sl2, -m));
        p1[u] = fast_exp2(fmaf(s[u][r + 1], sl2, -m));
        pf[2 * u + h][w] = pack_bf16x2(p0[u], p1[u]);
      }
      a[r] = p0[0];
      a[r + 1] = p1[0];
      if constexpr (NSUB >= 2) {
        a[r] += p0[1];
        a[r + 1] += p1[1];
      }
      if constexpr (NSUB == 4) {
        a[r] += p0[2] + p0[3];
        a[r + 1] += p1[2] + p1[3];
      }
    }
  }
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
    for (int r = 0; r < w; ++r) a[r] += a[r + w];
  ps = a[0];
}

// kMaybeEmpty: m may still be -inf on entry (every earlier stage of the row
// was fully masked, as block-sparse rows can be).  p is then formed against 0
// and the stage always refreshes.
template <int NSUB, bool kMaybeEmpty = false>
__device__ __forceinline__ void softmax_stage_stale(f32x16 (&s)[NSUB], int key0, int Skv, int g, float sl2,
                                                    float &m, float &lsum, f32x16 (&o)[4],
                                                    u32x4 (&pf)[2 * NSUB]) {
  // Both branches are rare (a stage that reaches past Skv, a refresh).  With
  // 64-key waves they are marked so (kHint), and the common path falls
  // through instead of branching around their code in every stage (measured
  // +0.4 % dense, +0.5 % 128x128 sparse); the 32-key waves of the key-split
  // kernel lost 3 % with that layout.  (The hint has to sit in the branch
  // condition itself.)
  constexpr bool kHint = NSUB >= 2;
  const bool past = key0 + 32 * NSUB > Skv;
  if (kHint ? __builtin_expect(past, 0) : past) mask_tail<NSUB>(s, key0, Skv, g);
  float ps;
  exp_pack_sum<NSUB>(s, sl2, kMaybeEmpty && m == kNegInf ? 0.f : m, pf, ps);
  // Two ballots OR'd on the scalar unit: one ballot of the lane-wise OR
  // compiles to a mask -> 0/1 -> compare round trip through VALU.
  uint64_t need = __builtin_amdgcn_ballot_w64(stage_sum_needs_refresh(ps));
  if constexpr (kMaybeEmpty) need |= __builtin_amdgcn_ballot_w64(m == kNegInf);
  const bool refresh = need != 0;
  if (kHint ? __builtin_expect(refresh, 0) : refresh) {
    const float mnew = fmaxf(m, tile_max<NSUB>(s, sl2));
    const float alpha = fast_exp2(m - (kMaybeEmpty && mnew == kNegInf ? 0.f : mnew));
    m = mnew;
    lsum *= alpha;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
    exp_pack_sum<NSUB>(s, sl2, kMaybeEmpty && m == kNegInf ? 0.f : m, pf, ps);
  }
  lsum += ps;
}

// Phase profile of the ping-pong kernels (H3A_PROFILE builds; every method
// compiles to nothing otherwise).  Workgroup 0's 8 waves each sum
// s_memtime ticks (the shader clock) per phase of their stage loop, in
// registers, and store them once after the loop, one row per wave (with
// dynamic dispatch, for the last work item workgroup 0 ran):
//   [0] DMA issue, and the loop's own branch   [1] first cluster
//   [2] mid-stage barrier                       [3] second cluster
//   [4] wait for the DMA (vmcnt)                [5] end-of-stage barrier
//   [6] stages run                              [7] loop, s_memtime ticks
//   [8] loop, s_memrealtime ticks (100 MHz)     [9] epilogue (normalise, store)
//   [10] prologue (work item start to loop start)
// Group A's first cluster is its matrix cluster (QK^T and PV MFMAs, which are
// interleaved and cannot be timed apart) and its second the softmax; group B
// the other way round.  Phases [0]-[5] tile the loop: their sum is [7].
constexpr int kProfSlots = H3A_PROF_SLOTS;
static_assert(H3A_PROF_WAVES == 8, "one row per wave of the dense workgroup");
__device__ unsigned long long g_prof[H3A_PROF_WAVES][kProfSlots];

struct PhaseClock {
  uint32_t ph[kProfSlots];  // a phase sums < 2^32 ticks for any stage count here
  uint64_t last, t_loop, rt_loop;
  bool on;
  __device__ __forceinline__ void begin(bool enabled) {
    if constexpr (H3A_PROFILE) {
      on = enabled;
#pragma unroll
      for (int i = 0; i < kProfSlots; ++i) ph[i] = 0;  // [7]-[10] are assigned, not summed
      last = __builtin_amdgcn_s_memtime();
    }
  }
  // Ticks since the previous mark go to phase i.  A mark is a scheduling
  // fence, so each phase holds exactly the code written between its marks
  // (s_memtime depends on nothing, and the scheduler would otherwise move it
  // among the MFMAs of a cluster).
  __device__ __forceinline__ void mark(int i) {
    if constexpr (H3A_PROFILE) {
      __builtin_amdgcn_sched_barrier(0);
      const uint64_t t = __builtin_amdgcn_s_memtime();
      ph[i] += (uint32_t)(t - last);
      last = t;
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __device__ __forceinline__ void loop_begin() {
    if constexpr (H3A_PROFILE) {
      t_loop = __builtin_amdgcn_s_memtime();
      ph[10] = (uint32_t)(t_loop - last);
      last = t_loop;
      rt_loop = __builtin_amdgcn_s_memrealtime();
    }
  }
  __device__ __forceinline__ void stage_done() {
    if constexpr (H3A_PROFILE) ph[6] += 1;
  }
  __device__ __forceinline__ void loop_end() {
    if constexpr (H3A_PROFILE) {
      ph[7] = (uint32_t)(last - t_loop);
      ph[8] = (uint32_t)(__builtin_amdgcn_s_memrealtime() - rt_loop);
      last = __builtin_amdgcn_s_memtime();
    }
  }
  // After the epilogue's stores: phase 9, then one row per wave to g_prof.
  __device__ __forceinline__ void finish(int wave, int lane) {
    if constexpr (H3A_PROFILE) {
      if (on) {
        ph[9] = (uint32_t)(__builtin_amdgcn_s_memtime() - last);
        if (lane == 0)
#pragma unroll
          for (int i = 0; i < kProfSlots; ++i) g_prof[wave][i] = ph[i];
      }
    }
  }
};

// Pin values to this point of the program: an empty volatile asm that reads
// and rewrites them.  Everything they depend on must be computed before it,
// and volatile asm keeps its place relative to the workgroup barriers.  Without
// it the compiler sinks softmax arithmetic (exp2, packing, the row sum) past a
// barrier toward the MFMAs that consume it, into the other cluster's slot.
__device__ __forceinline__ void pin(float &x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(u32x4 &x) { asm volatile("" : "+v"(x)); }

// Workgroup barrier that the instruction scheduler does not move work across.
__device__ __forceinline__ void slot_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
}

// The boundary between the two clusters of a ping-pong stage: a workgroup
// barrier when kNeeded (the block-sparse kernels: there group B waits for its
// own fetch right before it, and the barrier is what makes every wave's fetch
// visible to the group's next matrix cluster), otherwise only a scheduling
// fence (dense: the end-of-stage barrier alone keeps the groups one cluster
// apart once each softmax slot carries half of the fetch).
template <bool kNeeded>
__device__ __forceinline__ void mid_barrier() {
  if constexpr (kNeeded) {
    slot_barrier();
  } else {
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Dense ping-pong kernel: 8 waves x 32 query rows (one 256-row query tile per
// workgroup); waves 0-3 (group A) and 4-7 (group B) sit one of each per SIMD.
// Every stage of BN = 32*NSUB keys is split into a matrix-core cluster,
// MFMA(j): S(j+1) = K(j+1) Q^T and O += V(j) P(j), and a softmax cluster,
// SOFT(j): S(j+1) -> P(j+1).  Group B runs one cluster behind group A, so on
// every SIMD one wave issues MFMAs while the other issues the softmax's VALU
// work and the two pipes overlap.  A workgroup barrier ends every stage (and,
// in the block-sparse kernels, also separates its two clusters).
//
// Slots of stage j after the prologue:
//   slot 2j+1:  A: MFMA(j)                        B: DMA K(j+2), SOFT(j-1)
//   slot 2j+2:  A: DMA V(j+1), SOFT(j), wait      B: MFMA(j), wait
// K(j+2) goes to kbuf[j&1] and V(j+1) to vbuf[(j+1)&1]: group B fetches K and
// group A fetches V, each at the top of its softmax cluster, so each softmax
// slot carries half of the fetch.  Those buffers were last read by
// MFMA(j-1), which both groups finished before the barrier that ended stage
// j-1; the data is read by MFMA(j+1) in stage j+1, after every wave waited
// for its share of the fetch before the barrier that ends stage j.
//
// kSparse: block-sparse attention over pairs of query blocks.  Group A takes
// query block 2p and group B block 2p+1 of pair p, each with its own LUT row
// and its own double-buffered K/V stages in LDS; both step through the longer
// of the two stage lists (the shorter one's extra stages load nothing and are
// fully masked).  A group fetches its stages by LDS DMA, one instruction at a
// time spread over the PV MFMAs of its own matrix cluster (DmaSeq):
//   slot 2j+1:  A: MFMA(j) + DMA K(j+2), V(j+1)   B: SOFT(j-1), wait
//   slot 2j+2:  A: SOFT(j), wait                  B: MFMA(j) + DMA K(j+2), V(j+1)
// Both go to kbuf[j&1] and vbuf[(j+1)&1], last read by the group's own
// MFMA(j-1) before an earlier barrier; a wave waits for its own DMA before
// the barrier that precedes the group's MFMA(j+1).
//
// kKeySplit (with kSparse): pairs of 64-row query blocks.  Each group's 4
// waves are 2 query slices (32 rows) x 2 key halves: wave (rq, kh) scores its
// 32 rows against keys 32*kh .. 32*kh+31 of every 64-key stage (one 32-key
// score sub-tile, 16 MFMAs per stage) with its own running max, row sum and
// O; after the loop the key-half-1 wave hands (O, m, l) to its partner
// through LDS, which merges them as the split-tail combine does.
// The next work item from the per-XCD queues (see take_item_with) for a
// workgroup on XCD xcc, counters at `sched`.
__device__ __forceinline__ int take_item(int *sched, int whole, int pieces, int xcc) {
  return take_item_with(
      whole, pieces, xcc,
      [&](int x) { return __hip_atomic_load(sched + x * kQueueStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); },
      [&](int x) {
        return __hip_atomic_fetch_add(sched + x * kQueueStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      });
}

template <class L, int NSUB, bool kSparse>
struct PingPongLds {
  static constexpr int kKE = StageBytes<L, 32 * NSUB>::kK / 2;  // elements
  static constexpr int kVE = StageBytes<L, 32 * NSUB>::kV / 2;
  static constexpr int NG = kSparse ? 2 : 1;  // K/V streams: one per group (sparse)
  uint16_t k[NG][2][kKE];
  uint16_t v[NG][2][kVE];
};

// One work item of attn_fwd_pingpong_kernel: a 256-row query tile, a key
// range of a split tile, or (sparse) a pair of query blocks or a piece of one.
// `remapped`: the item number is already XCD-aware (taken from the queues),
// so whole tiles are not remapped.
template <class L, int NSUB, bool kSparse, bool kKeySplit, bool kWideKV, bool kTileMask>
__device__ __forceinline__ void pingpong_item(const AttnArgs &a, const int item, const bool remapped,
                                              PingPongLds<L, NSUB, kSparse> &lds, PhaseClock &pc) {
  constexpr int NW = 8;
  constexpr int BN = 32 * NSUB;  // keys per stage
  constexpr int WS = kKeySplit ? 1 : NSUB;  // 32-key score sub-tiles per wave and stage
  constexpr int QB = kKeySplit ? 64 : 128;  // sparse: query rows per group
  constexpr int kKE = PingPongLds<L, NSUB, kSparse>::kKE, kVE = PingPongLds<L, NSUB, kSparse>::kVE;
  static_assert(!kSparse || BN == kBN, "block-sparse stages are 64 keys");
  static_assert(!kKeySplit || (kSparse && NSUB == 2), "key-split pairs are block-sparse, 64-key stages");
  static_assert(!kTileMask || kKeySplit, "tile masks run on the key-split pairs");
  auto &kbuf_all = lds.k;
  auto &vbuf_all = lds.v;

  const int tid = threadIdx.x, wave = tid >> 6;
  // Opaque to the compiler, so nothing computed from the lane index is hoisted
  // out of the kernel's work-item loop to stay live through the stage loop.
  int lane = tid & 63;
  asm volatile("" : "+v"(lane));
  const int g = lane >> 5, l32 = lane & 31;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const bool lead = wave_u < NW / 2;  // group A
  const int grp = kSparse ? (lead ? 0 : 1) : 0;
  uint16_t(*kbuf)[kKE] = kbuf_all[grp];
  uint16_t(*vbuf)[kVE] = vbuf_all[grp];
  const int nstages = (a.Skv + BN - 1) / BN;
  // Work item of this workgroup.  With a split tail, the first
  // a.split_first items are whole query tiles; each later tile is cut into
  // a.split_pieces contiguous ranges of stages, one per workgroup, whose
  // partial results are merged by split_combine_kernel.
  // Sparse pairs split the same way, each piece taking the same fraction of
  // each group's own stage list (split_part).
  int w, piece = -1, j0 = 0, niter = nstages, split_part = -1;
  if (kSparse && item >= a.split_first) {
    piece = item - a.split_first;
    w = a.split_first + piece / a.split_pieces;
    split_part = piece % a.split_pieces;
  } else if (kSparse || item < a.split_first) {
    const int whole = a.split_first < a.total ? a.split_first : a.total;
    w = remapped ? item : xcd_remap(item, whole);
  } else {
    piece = item - a.split_first;
    w = a.split_first + piece / a.split_pieces;
    const int p = piece % a.split_pieces;
    j0 = (int)((int64_t)nstages * p / a.split_pieces);
    niter = (int)((int64_t)nstages * (p + 1) / a.split_pieces) - j0;  // >= 1
  }
  // Sparse: a.nqt counts query sub-blocks of QB rows and w runs over (b, h, pair).
  const int nw_bh = kSparse ? (a.nqt + 1) / 2 : a.nqt;
  const int qt = w % nw_bh, bh = w / nw_bh;
  const int h = bh % a.H, b = bh / a.H;
  const uint16_t *Qb = a.q + b * a.qsb + h * a.qsh;
  const uint16_t *Kb = a.k + b * a.ksb + h * a.ksh;
  const uint16_t *Vb = a.v + b * a.vsb + h * a.vsh;
  uint16_t *Ob = a.o + b * a.osb + h * a.osh;
  // Key-split: wave (rq, kh) of its group (see above); otherwise rq is the
  // wave's 32-row slice of the group's block and kh = 0.
  const int rq = kKeySplit ? (wave_u & 1) : (wave_u & 3);
  const int kh = kKeySplit ? ((wave_u >> 1) & 1) : 0;
  // Sparse: the pair's query sub-blocks, this group's (qb) and the other
  // group's (qo): 2qt and 2qt+1, or (tile path) the pair map's, clamped into
  // [0, nqt] (sub-block nqt is past the end: no rows, no stages).
  int qb = 2 * qt + grp, qo = 2 * qt + 1 - grp;
  if constexpr (kTileMask) {
    if (a.pair_map) {
      typedef const __attribute__((address_space(4))) int32_t *ConstInts;
      const ConstInts pm = (ConstInts)a.pair_map + 2 * (int64_t)w;
      const int m0 = pm[0], m1 = pm[1];
      const int s0 = m0 < 0 ? 0 : (m0 > a.nqt ? a.nqt : m0);
      const int s1 = m1 < 0 ? 0 : (m1 > a.nqt ? a.nqt : m1);
      qb = grp ? s1 : s0;
      qo = grp ? s0 : s1;
    }
  }
  const int qrow = kSparse ? qb * QB + rq * 32 + l32 : qt * 256 + wave * 32 + l32;
  // Sparse: this group's stage count and LUT row; both groups run the longer
  // of the two lists.  A piece of a split pair runs stages [gj0, gj0 + ngrp)
  // of the group's list.
  int ngrp = niter, gj0 = 0;
  const int32_t *lut_row = nullptr;
  int e_pre[4] = {0, 0, 0, 0};
  // Tile masks: stage j of a group is entries 2j and 2j+1 of its LUT row,
  // two 32-key columns; the waves of key half kh take entry 2j + kh (their
  // own column: its fetch, scores and mask).  ntile is the row's entry count.
  int ntile = 0;
  const uint32_t smag = stage_magic(a.sub);  // block_of_stage_magic(t, smag) = t / a.sub
  if constexpr (kSparse) {
    // Query sub-block qb reads LUT row qb / a.qmul (blk_q = 256: the two
    // 128-row blocks of a pair share one row; blk_q = 192: three 64-row ones).
    // The counts and the LUT are read through the constant address space:
    // they are not written during the kernel, so these stay scalar loads
    // after an earlier work item's stores (a global pointer would have to be
    // re-read per lane).  Both counts and the LUT entries of the first four
    // stages are loaded up front, unconditionally (indices clamped into their
    // rows), so that one wait covers them all: for a whole pair (no split)
    // stage j's entry is entry block_of_stage(j) of the row, and an entry at
    // or past the end of the list is never used (its stage's key is Skv).
    typedef const __attribute__((address_space(4))) int32_t *ConstInts;
    const ConstInts crow = (ConstInts)a.counts + (int64_t)bh * a.nqb;
    const int cnt_own = crow[(qb < a.nqt ? qb : 0) / a.qmul];
    const int cnt_oth = crow[(qo < a.nqt ? qo : 0) / a.qmul];
    lut_row = a.lut + ((int64_t)bh * a.nqb + (qb < a.nqt ? qb : 0) / a.qmul) * a.lut_stride;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = kTileMask ? 2 * j + kh : block_of_stage_magic(j, smag);
      e_pre[j] = ((ConstInts)lut_row)[e < a.lut_stride ? e : a.lut_stride - 1];
    }
    auto stages_of = [&](int qb, int cnt) __attribute__((always_inline)) -> int {
      if (qb >= a.nqt) return 0;
      const int n = cnt < 0 ? 0 : (cnt > a.lut_stride ? a.lut_stride : cnt);
      return kTileMask ? (n + 1) / 2 : n * a.sub;
    };
    if constexpr (kTileMask)
      ntile = qb >= a.nqt ? 0 : (cnt_own < 0 ? 0 : (cnt_own > a.lut_stride ? a.lut_stride : cnt_own));
    auto part_of = [&](int n, int &first) __attribute__((always_inline)) -> int {
      if (split_part < 0) {
        first = 0;
        return n;
      }
      first = (int)((int64_t)n * split_part / a.split_pieces);
      return (int)((int64_t)n * (split_part + 1) / a.split_pieces) - first;
    };
    int other_j0;
    ngrp = part_of(stages_of(qb, cnt_own), gj0);
    const int nother = part_of(stages_of(qo, cnt_oth), other_j0);
    niter = ngrp > nother ? ngrp : nother;
  }
  // Sparse: LUT entry of local stage j (a key block of a.sub stages; read
  // through the constant address space, so it is a scalar load), and the
  // stage's first key from it.  Past this group's last stage, and for LUT
  // entries that name no key block, the key is Skv, which loads nothing.
  // Both are branch-free scalar code (stage_magic, selects): they run in the
  // softmax slots of every stage.  The entry index is clamped into the
  // group's part of the row (entry 0 for an empty list, whose keys are all
  // Skv whatever the entry).
  auto lut_entry = [&](int j) __attribute__((always_inline)) -> int {
    if constexpr (kSparse) {
      const __attribute__((address_space(4))) int32_t *row =
          (const __attribute__((address_space(4))) int32_t *)lut_row;
      const int jc = j < ngrp ? j : ngrp - 1;
      if constexpr (kTileMask) {
        const int i = 2 * (jc > 0 ? jc : 0) + kh;
        return row[i < a.lut_stride ? i : a.lut_stride - 1];
      } else {
        return row[block_of_stage_magic(gj0 + (jc > 0 ? jc : 0), smag)];
      }
    } else {
      return 0;
    }
  };
  // Tile masks: an entry is column << 8 | mask, the column in units of 32
  // keys (a.blk_k = 32, a.sub = 1); an arithmetic shift keeps a negative
  // entry negative, so it still names no key block.  Past the row's entries
  // (the last stage can hold one column) the key is Skv.
  auto key_of_entry = [&](int j, int e) __attribute__((always_inline)) -> int {
    if constexpr (kSparse) {
      const int kb = kTileMask ? (e >> 8) : e;
      // Two equivalent forms; each measured faster in one kernel (the
      // arithmetic one +0.5 % in the 128-row pairs, the select one +0.6 % in
      // the key-split pairs), through the code layout around them.
      const int key0 = kKeySplit ? lut_stage_key0_sel(gj0 + j, kb, a.nkb, a.blk_k, a.sub, smag, a.Skv)
                                 : lut_stage_key0_magic(gj0 + j, kb, a.nkb, a.blk_k, a.sub, smag, a.Skv);
      if constexpr (kTileMask) return j < ngrp && 2 * j + kh < ntile ? key0 : a.Skv;
      else return j < ngrp ? key0 : a.Skv;
    } else {
      return j < niter ? (j0 + j) * BN : a.Skv;
    }
  };
  auto key_base = [&](int j) __attribute__((always_inline)) -> int { return key_of_entry(j, lut_entry(j)); };
  // The same for the prologue's stages 0-3, from the entries loaded up front.
  auto pro_entry = [&](int j) __attribute__((always_inline)) -> int {
    if constexpr (kSparse) return split_part < 0 ? e_pre[j] : lut_entry(j);
    else return 0;
  };
  auto pro_key = [&](int j) __attribute__((always_inline)) -> int { return key_of_entry(j, pro_entry(j)); };
  if (kSparse && niter == 0) {
    // Neither query block of the pair keeps a key block (in this piece): O = 0,
    // or an empty partial result (m = -inf, l = 0, O = 0).
    if (piece >= 0) {
      const int row = wave * 32 + l32;
      float *po = a.ws + ((int64_t)piece * 256 + row) * kD + 4 * g;
#pragma unroll
      for (int c = 0; c < 16; ++c) *(float4 *)(po + 8 * c) = float4{0.f, 0.f, 0.f, 0.f};
      if (g == 0) {
        float *pml = a.ws + (int64_t)(a.total - a.split_first) * 256 * kD + ((int64_t)piece * 256 + row) * 2;
        *(float2 *)pml = float2{kNegInf, 0.f};
      }
      return;
    }
    if (qrow < a.Sq && kh == 0) {
      uint16_t *p = Ob + (int64_t)qrow * a.oss + 4 * g;
#pragma unroll
      for (int c = 0; c < 16; ++c) *(u32x2 *)(p + 8 * c) = u32x2{0, 0};
    }
    return;
  }

  // Global loads: as flat loads they would also count as LDS/scalar accesses
  // and hold up the next wait for those.
  u32x4 qf[8];
  if (qrow < a.Sq) {
    const uint16_t *p = Qb + (int64_t)qrow * a.qss + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = *(const __attribute__((address_space(1))) u32x4 *)(p + ks * 16);
  } else {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = u32x4{0, 0, 0, 0};
  }
  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{0.f};
  float m = kNegInf;  // running row max, in scale*log2(e) units
  float lsum = 0.f;   // this lane's share of the running row sum
  // Key half kh starts 32 rows into the stage (an offset that neither layout's
  // per-step offsets interact with).
  const int k_rd = L::k_base(l32, g) + kh * 32 * L::kKRow;
  const int v_rd = L::v_base(lane) + kh * 32 * L::kVRow;

  // K/V stages are fetched by LDS DMA, the 4 waves of a group each issuing
  // the instructions of one column of the 4-wave layout (TileDma).  Dense:
  // group B fetches the K stages and group A the V stages (waves w and w+4
  // share a column), each at the top of its softmax slot.  Sparse: each
  // group fetches its own K/V stream, spread over its matrix cluster.
  // Tile masks: each key half of a stage is its own 32-key column, fetched by
  // the two waves of that half (rq = 0, 1) into rows 32*kh .. 32*kh+31.
  using KDma = std::conditional_t<kTileMask, TileDma<2, L, false, 32>, TileDma<NW / 2, L, false, BN>>;
  using VDma = std::conditional_t<kTileMask, TileDma<2, L, true, 32>, TileDma<NW / 2, L, true, BN>>;
  KDma kdma;
  VDma vdma;
  kdma.init(a.kss, kTileMask ? rq : (wave_u & 3), lane);
  vdma.init(a.vss, kTileMask ? rq : (wave_u & 3), lane);
  static_assert(!kTileMask || (KDma::kInst == 4 && VDma::kInst == 4), "4 loads of each stream per wave and stage");
  auto kdst = [&](uint16_t *buf) __attribute__((always_inline)) {
    return kTileMask ? buf + kh * 32 * (L::kKRow / 2) : buf;
  };
  auto vdst = [&](uint16_t *buf) __attribute__((always_inline)) {
    return kTileMask ? buf + kh * 32 * (L::kVRow / 2) : buf;
  };
  constexpr int kKI = decltype(kdma)::kInst, kVI = decltype(vdma)::kInst;
  // Sparse stage fetches.  By default one descriptor per (b,h) slice, built
  // here, and each stage's byte offset added to the lanes' offsets: the
  // per-stage descriptor (a 64-bit base and a row count for the range check)
  // cost ~35 scalar instructions per stage.  Rows past Skv and stages past a
  // list (key Skv) fall outside the slice's range and load zeros, as with
  // the per-stage descriptors.  kWideKV: offsets up to (Skv + 64) rows would
  // pass 2^32 bytes, so every stage gets its own descriptor based on its
  // first row.
  constexpr bool kHeadDesc = kSparse && !kWideKV;
  const u32x4 kd_head = stage_desc(Kb, a.kss, a.Skv), vd_head = stage_desc(Vb, a.vss, a.Skv);
  const uint32_t krow_bytes = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a.kss * 2));
  const uint32_t vrow_bytes = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a.vss * 2));
  auto k_desc = [&](int key0) __attribute__((always_inline)) {
    if constexpr (kHeadDesc) return kd_head; else return kdma.desc(Kb, a.kss, key0, a.Skv);
  };
  auto v_desc = [&](int key0) __attribute__((always_inline)) {
    if constexpr (kHeadDesc) return vd_head; else return vdma.desc(Vb, a.vss, key0, a.Skv);
  };
  auto k_soff = [&](int key0) __attribute__((always_inline)) {
    return kHeadDesc ? (uint32_t)key0 * krow_bytes : 0u;
  };
  auto v_soff = [&](int key0) __attribute__((always_inline)) {
    return kHeadDesc ? (uint32_t)key0 * vrow_bytes : 0u;
  };
  // LDS operand reads issued ahead of a matrix cluster's first MFMA (then 2
  // after each MFMA), and the wave priority raised (s_setprio 1) during the
  // cluster: same-box sweeps chose 4 reads ahead for the dense kernel and the
  // 128-row pairs, 5 for the key-split pairs (16 MFMAs per cluster), and no
  // raise for the dense kernel.  In the block-sparse kernels group B raises
  // its priority during its matrix cluster while group A's cluster runs at
  // the default: group B's cluster, which shares its slot with group A's
  // softmax, otherwise ran ~15 % longer than group A's and bounded the stage.
  constexpr int kReadAhead = kKeySplit ? 5 : 4;
  constexpr int kReadsPerMfma = 2;
  constexpr bool kRaisePrio = kSparse;

  // Dense: cursors of the K stream at local stage 2 and the V stream at
  // stage 1, where the loop's fetches start.  The range ends at key_end, so
  // stages from niter on load nothing, as key_base(j >= niter) = Skv does.
  StageCursor<BN> kcur, vcur;
  if constexpr (!kSparse) {
    const int key_end = a.Skv < (j0 + niter) * BN ? a.Skv : (j0 + niter) * BN;
    kcur.init(Kb, a.kss, (j0 + 2) * BN, key_end);
    vcur.init(Vb, a.vss, (j0 + 1) * BN, key_end);
  }

  // Prologue, all waves in step: K(0), V(0), K(1) in; S(0); P(0).  Dense:
  // group B fetches the K stages, group A the V stage.
  const int pkey0 = pro_key(0), pkey1 = pro_key(1);
  const uint32_t pmask0 = kTileMask ? (uint32_t)pro_entry(0) & 0xffu : 0u;
  if constexpr (kSparse) {
    kdma.issue(Kb, a.kss, pkey0, a.Skv, kdst(kbuf[0]));
    vdma.issue(Vb, a.vss, pkey0, a.Skv, vdst(vbuf[0]));
    kdma.issue(Kb, a.kss, pkey1, a.Skv, kdst(kbuf[1]));
  } else if (lead) {
    vdma.issue(Vb, a.vss, pkey0, a.Skv, vbuf[0]);
  } else {
    kdma.issue(Kb, a.kss, pkey0, a.Skv, kbuf[0]);
    kdma.issue(Kb, a.kss, pkey1, a.Skv, kbuf[1]);
  }
  wait_vmem_all();
  __syncthreads();
  f32x16 s[WS];
  u32x4 pf[2 * WS];
  score_tile<L, WS>(kbuf[0], qf, k_rd, s);
  if constexpr (kTileMask) apply_tile_mask<WS>(s, pmask0, rq, l32);
  softmax_stage<WS>(s, pkey0 + (kTileMask ? 0 : 32 * kh), a.Skv, g, a.sl2, m, lsum, o, pf);
  __syncthreads();  // kbuf[0] is free for K(2)

  // Dense, stage j's fetch from the stream cursors: group A's V(j+1) into
  // vbuf[(j+1)&1], group B's K(j+2) into kbuf[j&1].
  auto dma_v = [&](auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;  // j & 1
    vdma.template issue_desc<0, kVI>(vcur.desc(), vbuf[P ^ 1]);
    vcur.advance();
  };
  auto dma_k = [&](auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;  // j & 1
    kdma.template issue_desc<0, kKI>(kcur.desc(), kbuf[P]);
    kcur.advance();
  };
  // Sparse: entering stage j the group holds the first keys of stages j, j+1
  // and j+2 and the LUT entry of stage j+3.  stage_keys(j) takes stage j's
  // keys (K(j+2), V(j+1), the softmax mask) and moves the window on;
  // lut_next(j), issued after a barrier, loads the entry of stage j+4 for
  // the next stage_keys, so the scalar load's wait falls on the following
  // barrier with a softmax cluster in between.  The softmax masks with a
  // held key too: stage j+1's for group A (SOFT(j)), stage j's for group B
  // (SOFT(j-1)).  Tile masks travel with the keys (mw0..mw2, soft_mask).
  int kw0 = pkey0, kw1 = pkey1, kw2 = pro_key(2), e3 = pro_entry(3);
  int soft_key = 0;
  int key_k = 0, key_v = 0;
  uint32_t mw0 = pmask0, mw1 = 0, mw2 = 0, soft_mask = 0;
  if constexpr (kTileMask) {
    mw1 = (uint32_t)pro_entry(1) & 0xffu;
    mw2 = (uint32_t)pro_entry(2) & 0xffu;
  }
  auto stage_keys = [&](int j) __attribute__((always_inline)) {
    soft_key = lead ? kw1 : kw0;
    key_k = kw2;
    key_v = kw1;
    const int kw3 = key_of_entry(j + 3, e3);
    kw0 = kw1;
    kw1 = kw2;
    kw2 = kw3;
    if constexpr (kTileMask) {
      soft_mask = lead ? mw1 : mw0;
      mw0 = mw1;
      mw1 = mw2;
      mw2 = (uint32_t)e3 & 0xffu;
    }
  };
  auto lut_next = [&](int j) __attribute__((always_inline)) { e3 = lut_entry(j + 4); };
  static_assert(!kSparse || (decltype(kdma)::kInstTotal % (NW / 2) == 0 &&
                             decltype(vdma)::kInstTotal % (NW / 2) == 0),
                "every wave issues the same number of DMA loads per stage");
  // The score and PV MFMAs of the cluster with the LDS operand reads issued
  // ahead of them: kReadAhead up front, then kReadsPerMfma after each MFMA,
  // so every read is in flight for several MFMAs.
  auto order_reads = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_group_barrier(0x100, kReadAhead, 0);
#pragma unroll
    for (int i = 0; i < 16 * WS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, kReadsPerMfma, 0);
    }
  };
  // Dense matrix cluster: one basic block of 16*NSUB MFMAs (the last stage's
  // scores are of the zero tile past the keys and are discarded).
  auto mfma = [&](auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    if (kRaisePrio) __builtin_amdgcn_s_setprio(1);
    score_tile<L, WS>(kbuf[P ^ 1], qf, k_rd, s);
    pv_tile<L, 2 * WS>(vbuf[P], pf, v_rd, o);
    order_reads();
    if (kRaisePrio) __builtin_amdgcn_s_setprio(0);
  };
  // Sparse matrix cluster with this wave's fetch of K(j+2) (kseq) and V(j+1)
  // (vseq) spread over it: all NK + NV instructions among the PV MFMAs, K
  // first, evenly spaced.  Each DMA instruction is volatile asm that touches
  // memory, so it keeps its place among the LDS operand reads, which the
  // scheduling groups interleave with the MFMAs.
  auto mfma_dma = [&](auto par, auto &kseq, auto &vseq) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    constexpr int NK = std::remove_reference_t<decltype(kseq)>::kCount;
    constexpr int NV = std::remove_reference_t<decltype(vseq)>::kCount;
    constexpr int NP = 4 * 2 * WS, NI = NK + NV;  // PV MFMAs, DMA instructions
    if (kRaisePrio && !lead) __builtin_amdgcn_s_setprio(1);
    score_tile<L, WS>(kbuf[P ^ 1], qf, k_rd, s);
    pv_tile<L, 2 * WS>(vbuf[P], pf, v_rd, o, [&](int t) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        if (t == i * NP / NI) {
          if (i < NK) kseq.issue(); else vseq.issue();
        }
      }
    });
    order_reads();
    if (kRaisePrio) __builtin_amdgcn_s_setprio(0);
  };
  // Sparse: the cluster with the group's fetch of K(j+2) and V(j+1) (keys
  // from stage_keys) into the buffers the group read in MFMA(j-1).
  auto mfma_fetch = [&](auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    DmaSeq<decltype(kdma)> kseq(kdma, k_desc(key_k), kdst(kbuf[P]), k_soff(key_k));
    DmaSeq<decltype(vdma)> vseq(vdma, v_desc(key_v), vdst(vbuf[P ^ 1]), v_soff(key_v));
    mfma_dma(par, kseq, vseq);
  };
  // Softmax cluster.  Its results are pinned to the slot (pin), so that the
  // compiler does not sink them past the barrier toward the MFMAs.
  auto soft = [&](int j) __attribute__((always_inline)) {
    // Tile masks: the keys are already this wave's own column's.
    const int key0 = (kSparse ? soft_key : key_base(j + 1)) + (kTileMask ? 0 : 32 * kh);
    if constexpr (kTileMask) apply_tile_mask<WS>(s, soft_mask, rq, l32);
    softmax_stage_stale<WS, kSparse>(s, key0, a.Skv, g, a.sl2, m, lsum, o, pf);
#pragma unroll
    for (int i = 0; i < 2 * WS; ++i) pin(pf[i]);
    pin(lsum);
    pin(m);
  };

  pc.loop_begin();
  if (lead) {
    auto stage = [&](auto par, int j) __attribute__((always_inline)) {
      if constexpr (kSparse) {
        pc.mark(0);
        stage_keys(j);
        mfma_fetch(par);
        pc.mark(1);
        mid_barrier<kSparse>();
        pc.mark(2);
        lut_next(j);
        if (j + 1 < niter) soft(j);
        pc.mark(3);
        wait_vmem_all();
        pc.mark(4);
        slot_barrier();
        pc.mark(5);
        pc.stage_done();
      } else {
        pc.mark(0);
        mfma(par);
        pc.mark(1);
        mid_barrier<kSparse>();
        pc.mark(2);
        dma_v(par);
        __builtin_amdgcn_sched_barrier(0);
        if (j + 1 < niter) soft(j);
        pc.mark(3);
        wait_vmem_all();
        pc.mark(4);
        slot_barrier();
        pc.mark(5);
        pc.stage_done();
      }
    };
    for (int j = 0; j < niter; j += 2) {
      stage(std::integral_constant<int, 0>{}, j);
      if (j + 1 < niter) stage(std::integral_constant<int, 1>{}, j + 1);
    }
  } else {
    // kFirst: stage 0, which has no softmax before its matrix cluster (P(0)
    // came from the prologue); peeled off so that the loop body has no branch.
    auto stage = [&](auto par, int j, auto first) __attribute__((always_inline)) {
      if constexpr (kSparse) {
        pc.mark(0);
        stage_keys(j);  // also sets the key SOFT(j-1) masks with: stage j's first
        lut_next(j);
        if constexpr (!decltype(first)::value) soft(j - 1);
        pc.mark(1);
        // This wave's fetch of K(j+1) and V(j), issued during MFMA(j-1).
        wait_vmem_all();
        pc.mark(4);
        mid_barrier<kSparse>();
        pc.mark(2);
        mfma_fetch(par);
        pc.mark(3);
        slot_barrier();
        pc.mark(5);
        pc.stage_done();
      } else {
        dma_k(par);
        pc.mark(0);
        if constexpr (!decltype(first)::value) soft(j - 1);
        pc.mark(1);
        mid_barrier<kSparse>();
        pc.mark(2);
        mfma(par);
        pc.mark(3);
        wait_vmem_all();
        pc.mark(4);
        slot_barrier();
        pc.mark(5);
        pc.stage_done();
      }
    };
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;
    stage(C0{}, 0, std::true_type{});
    for (int j = 1; j < niter; j += 2) {
      stage(C1{}, j, std::false_type{});
      if (j + 1 < niter) stage(C0{}, j + 1, std::false_type{});
    }
  }
  pc.loop_end();
  // Sparse: group B's last stage issued loads (of nothing: keys past its
  // list) into group B's K/V buffers that may still be in flight.  The
  // key-split exchange below writes those buffers from other waves, so there
  // every wave waits for its loads and a barrier follows.  Otherwise nothing
  // touches group B's buffers before this wave's next fetch into them, which
  // lands after these (a wave's loads complete in order), and the kernel
  // waits for them before it exits.
  if constexpr (kKeySplit) {
    wait_vmem_all();
    __syncthreads();
  }

  if constexpr (kKeySplit) {
    // Every LDS read and write of the stages is complete (the barrier
    // above), so a group's own K/V buffers hold the exchange: O of each
    // slice's key-half-1 wave in the K buffers (lane-major: 64 consecutive
    // floats per register), its m and l in the V buffers.
    static_assert(sizeof(kbuf_all[0]) >= 2 * 64 * 64 * sizeof(float), "O exchange fits a group's K buffers");
    static_assert(sizeof(vbuf_all[0]) >= 2 * 2 * 64 * sizeof(float), "m/l exchange fits a group's V buffers");
    float *xo = reinterpret_cast<float *>(&kbuf[0][0]) + rq * 64 * 64;
    float *xm = reinterpret_cast<float *>(&vbuf[0][0]) + rq * 2 * 64;
    if (kh == 1) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) xo[(16 * dt + r) * 64 + lane] = o[dt][r];
      xm[lane] = m;
      xm[64 + lane] = lsum;
    }
    __syncthreads();
    if (kh == 1) {  // no barrier follows
      pc.finish(wave, lane);
      return;
    }
    const float m2 = xm[lane], l2 = xm[64 + lane];
    const float mn = fmaxf(m, m2);
    const float a1 = m == kNegInf ? 0.f : fast_exp2(m - mn);
    const float a2 = m2 == kNegInf ? 0.f : fast_exp2(m2 - mn);
    lsum = lsum * a1 + l2 * a2;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] = o[dt][r] * a1 + xo[(16 * dt + r) * 64 + lane] * a2;
  }

  const float ltot = half_swap_sum(lsum);
  if (piece >= 0) {
    // Partial result of one key range: unnormalised O, the reference max m
    // it is relative to (scale*log2(e) units) and the row sum, for all 256
    // rows of the tile (rows past Sq included; the combine skips them).
    const int row = wave * 32 + l32;
    float *po = a.ws + ((int64_t)piece * 256 + row) * kD + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        *(float4 *)(po + dt * 32 + 8 * rr) =
            float4{o[dt][4 * rr + 0], o[dt][4 * rr + 1], o[dt][4 * rr + 2], o[dt][4 * rr + 3]};
    if (g == 0) {
      float *pml = a.ws + (int64_t)(a.total - a.split_first) * 256 * kD + ((int64_t)piece * 256 + row) * 2;
      *(float2 *)pml = float2{m, ltot};
    }
    pc.finish(wave, lane);
    return;
  }
  const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
  // The wave's normalised O (32 rows x 128 dims, bf16) leaves through LDS.
  // A lane holds 4-dim pieces of one row, so stored directly every
  // instruction would write 16 bytes into each of 32 rows; written into a
  // wave-private tile (256-byte rows, 16-byte chunks XOR-swizzled by row) and
  // read back a chunk per lane, every store writes 4 whole rows.  The tile is
  // free: key-split, the wave's own exchange slot, which it has read;
  // otherwise a quarter of group A's K or V buffers, whose fetches all
  // completed before the loop's last barrier (group B's last loads, still in
  // flight for other waves, only touch group B's buffers).
  {
    uint8_t *tile;
    if constexpr (kKeySplit) {
      tile = reinterpret_cast<uint8_t *>(&kbuf[0][0]) + rq * (64 * 64 * 4);
    } else {
      tile = (wave_u < 4 ? reinterpret_cast<uint8_t *>(&kbuf_all[0][0][0])
                         : reinterpret_cast<uint8_t *>(&vbuf_all[0][0][0])) + (wave_u & 3) * (32 * 256);
    }
    static_assert(sizeof(kbuf_all[0]) >= 4 * 32 * 256 && sizeof(vbuf_all[0]) >= 4 * 32 * 256,
                  "four O tiles fit group A's K buffers and its V buffers");
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const u32x2 val = {pack_bf16x2(o[dt][4 * rr + 0] * inv, o[dt][4 * rr + 1] * inv),
                           pack_bf16x2(o[dt][4 * rr + 2] * inv, o[dt][4 * rr + 3] * inv)};
        const int c = 4 * dt + rr;  // 16-byte chunk of the row: dims 8c .. 8c+7
        *(u32x2 *)(tile + l32 * 256 + ((c ^ (l32 & 15)) << 4) + 8 * g) = val;
      }
    }
    // Buffer stores over the wave's valid rows: rows past Sq fall outside the
    // resource and are dropped, so no store sits behind a branch (and a
    // later vmcnt wait can count exactly the stores issued).
    const int q0 = __builtin_amdgcn_readfirstlane(qrow - l32), ch = lane & 15;
    const int nrows = a.Sq - q0 < 32 ? a.Sq - q0 : 32;
    const __amdgpu_buffer_rsrc_t ores = stage_rsrc(Ob + (int64_t)q0 * a.oss, a.oss, nrows);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 4 * i + (lane >> 4);
      const u32x4 val = *(const u32x4 *)(tile + r * 256 + ((ch ^ (r & 15)) << 4));
      __builtin_amdgcn_raw_buffer_store_b128(val, ores, (int)((uint32_t)r * (uint32_t)a.oss * 2u + 16u * ch), 0, 0);
    }
  }
  pc.finish(wave, lane);
}

template <class L, int NSUB, bool kSparse = false, bool kKeySplit = false, bool kWideKV = false,
          bool kTileMask = false>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
attn_fwd_pingpong_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) PingPongLds<L, NSUB, kSparse> lds;
  __shared__ int next_item;
  PhaseClock pc;
  // Static dispatch (a.sched null): work item blockIdx.x.  Dynamic dispatch:
  // a persistent grid whose workgroups take items from the queues until all
  // are empty; the barriers around the take keep every wave of the previous
  // item clear of the LDS before the next item's first fetch lands there.
  // Each item reads the arguments afresh from the kernarg segment, through a
  // pointer the compiler cannot follow across iterations: kept in SGPRs over
  // the whole loop instead, they push the stage loop's register allocation
  // into waiting for every LDS operand read (lgkmcnt(0) before each MFMA).
  // With one item per workgroup the loop runs once.
  typedef const __attribute__((address_space(4))) AttnArgs *KernargPtr;
  for (int item = blockIdx.x;;) {
    KernargPtr kp = (KernargPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(kp));
    static_assert(sizeof(AttnArgs) % 4 == 0, "kernel arguments copied as words");
    typedef const __attribute__((address_space(4))) uint32_t *KernargWords;
    uint32_t words[sizeof(AttnArgs) / 4];
#pragma unroll
    for (int i = 0; i < (int)(sizeof(AttnArgs) / 4); ++i) words[i] = ((KernargWords)kp)[i];
    AttnArgs args;
    __builtin_memcpy(&args, words, sizeof(args));
    if (args.sched) {
      // A take is an agent-scope atomic's round trip, about 3000 shader
      // cycles under load.  Issued during the work item's prologue or right
      // after its stage loop instead, it measured as fast or slower for
      // every kernel.
      __syncthreads();
      if (threadIdx.x == 0) {
        const int xcc = (int)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & (kQueues - 1));  // XCC_ID
        const int whole = args.split_first < args.total ? args.split_first : args.total;
        next_item = take_item(args.sched, whole, args.total - whole, xcc);
      }
      __syncthreads();
      item = __builtin_amdgcn_readfirstlane(next_item);
      if (item < 0) break;
    }
    pc.begin(blockIdx.x == 0);
    pingpong_item<L, NSUB, kSparse, kKeySplit, kWideKV, kTileMask>(args, item, args.sched != nullptr, lds, pc);
    KernargPtr kq = (KernargPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(kq));
    if (!kq->sched) break;
  }
  // The last work item's trailing loads (see pingpong_item) land before the
  // workgroup ends and its LDS is released.
  if constexpr (kSparse) wait_vmem_all();
}

// Clears the dispatch queues' counters before a dynamic launch (a kernel, not
// a memset, so the pair can be captured in a graph).
__global__ void __launch_bounds__(256) sched_clear_kernel(int *sched) {
  if (threadIdx.x < kQueues * kQueueStride) sched[threadIdx.x] = 0;
}

// Merge the key-range pieces of the split tiles:
//   O = sum_p 2^(m_p - M) O_p / sum_p 2^(m_p - M) l_p,  M = max_p m_p.
// One thread per (split tile, row, 4 dims); 8 rows per 256-thread block.
__global__ void __launch_bounds__(256) split_combine_kernel(AttnArgs a) {
  const int ntiles = (a.total - a.split_first) / a.split_pieces;
  const int64_t item = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);  // (split tile, row)
  if (item >= (int64_t)ntiles * 256) return;
  const int t = (int)(item / 256), row = (int)(item % 256), d = 4 * (threadIdx.x & 31);
  const int tile = a.split_first + t;
  const int tiles_bh = a.lut ? (a.nqt + 1) / 2 : a.nqt;  // sparse: pairs of 128-row blocks
  const int qt = tile % tiles_bh, bh = tile / tiles_bh;
  const int h = bh % a.H, b = bh / a.H;
  const int qrow = qt * 256 + row;
  if (qrow >= a.Sq) return;
  const int P = a.split_pieces;
  const float *ml = a.ws + (int64_t)(a.total - a.split_first) * 256 * kD;
  float M = kNegInf;
  for (int p = 0; p < P; ++p) M = fmaxf(M, ml[((int64_t)(t * P + p) * 256 + row) * 2]);
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
  for (int p = 0; p < P; ++p) {
    const int64_t pr = (int64_t)(t * P + p) * 256 + row;
    const float mp = ml[pr * 2], lp = ml[pr * 2 + 1];
    const float wgt = (mp == kNegInf) ? 0.f : fast_exp2(mp - M);
    const float4 op = *(const float4 *)(a.ws + pr * kD + d);
    acc.x = fmaf(wgt, op.x, acc.x);
    acc.y = fmaf(wgt, op.y, acc.y);
    acc.z = fmaf(wgt, op.z, acc.z);
    acc.w = fmaf(wgt, op.w, acc.w);
    L = fmaf(wgt, lp, L);
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint16_t *po = a.o + b * a.osb + h * a.osh + (int64_t)qrow * a.oss + d;
  *(u32x2 *)po = u32x2{pack_bf16x2(acc.x * inv, acc.y * inv), pack_bf16x2(acc.z * inv, acc.w * inv)};
}

// ---------------------------------------------------------------------------
// Fragment tests: one wave, the same staging and fragment code as above.
__global__ void __launch_bounds__(64) test_qk_kernel(const uint16_t *Q, const uint16_t *K, float *S) {
  __shared__ __attribute__((aligned(16))) uint16_t kb[StageBytes<SwzLayout>::kK / 2];
  const int tid = threadIdx.x, g = tid >> 5, l32 = tid & 31;
  TileDma<1, SwzLayout, false> dma;
  dma.init(kD, 0, tid);
  dma.issue(K, kD, 0, kBN, kb);
  wait_vmem_all();
  __syncthreads();
  u32x4 qf[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) qf[ks] = *(const u32x4 *)(Q + l32 * kD + ks * 16 + 8 * g);
  f32x16 s[2];
  score_tile<SwzLayout, 2>(kb, qf, SwzLayout::k_base(l32, g), s);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int key = 8 * (r >> 2) + 4 * g + (r & 3);
    S[l32 * kBN + key] = s[0][r];
    S[l32 * kBN + key + 32] = s[1][r];
  }
}

__global__ void __launch_bounds__(64) test_pv_kernel(const uint16_t *P, const uint16_t *V, float *O) {
  __shared__ __attribute__((aligned(16))) uint16_t vb[StageBytes<SwzLayout>::kV / 2];
  const int tid = threadIdx.x, g = tid >> 5, l32 = tid & 31;
  TileDma<1, SwzLayout, true> dma;
  dma.init(kD, 0, tid);
  dma.issue(V, kD, 0, kBN, vb);
  wait_vmem_all();
  __syncthreads();
  // Place P[q][key] where the score accumulators would hold it.
  f32x16 s[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int key = 8 * (r >> 2) + 4 * g + (r & 3);
    s[0][r] = __uint_as_float((uint32_t)P[l32 * kBN + key] << 16);
    s[1][r] = __uint_as_float((uint32_t)P[l32 * kBN + key + 32] << 16);
  }
  u32x4 pf[4];
  pack_p<2>(s, pf);
  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{0.f};
  pv_tile<SwzLayout, 4>(vb, pf, SwzLayout::v_base(tid), o);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[l32 * kD + dt * 32 + 8 * (r >> 2) + 4 * g + (r & 3)] = o[dt][r];
}

// ---------------------------------------------------------------------------
// Block map [B,H,nq,nk] (0/1 bytes) -> ascending LUT + counts, one thread per row.
__global__ void __launch_bounds__(256) block_map_to_lut_kernel(const uint8_t *map, int64_t rows,
                                                               int nk, int32_t *lut,
                                                               int32_t *counts, int max_k) {
  const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const uint8_t *m = map + row * nk;
  int32_t *out = lut + row * max_k;
  int c = 0;
  for (int j = 0; j < nk; ++j) {
    if (m[j] != 0) {
      if (c < max_k) out[c] = j;
      ++c;
    }
  }
  const int kept = c < max_k ? c : max_k;
  for (int j = kept; j < max_k; ++j) out[j] = -1;
  counts[row] = kept;
}

// ---------------------------------------------------------------------------
// Pairs of 64-row query sub-blocks for the tile path.  A pair runs as many
// stages as the longer of its two lists, so a pair of unequal lists leaves
// one group idle for the difference: with blk_q 80, 96, 112, 144, ... a block
// boundary falls inside some sub-blocks and not others, and those hold the
// union of two blocks' lists.  One workgroup per (b,h) sorts its sub-blocks
// by stage count, descending (ties by index), in LDS (bitonic), and pairs
// neighbours: map[bh][p] = sorted entries 2p and 2p+1, an odd count pairing
// the last with sub-block nsub, which has no rows.  Which sub-blocks share a
// workgroup does not change any row's arithmetic.
__global__ void __launch_bounds__(1024) tile_pair_map_kernel(const int32_t *counts, int nsub, int lut_stride,
                                                             int32_t *map) {
  __shared__ uint32_t key[kPairSortMax];
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.x;
  int n = 2;
  while (n < nsub) n <<= 1;
  const int32_t *c = counts + bh * nsub;
  for (int i = tid; i < n; i += 1024) {
    uint32_t kv = 0xffffffffu;  // padding sorts last
    if (i < nsub) {
      const int e = c[i] < 0 ? 0 : (c[i] > lut_stride ? lut_stride : c[i]);
      const uint32_t st = (uint32_t)(e + 1) / 2;  // stages, <= 32767
      kv = ((0x7fffu - st) << 16) | (uint32_t)i;
    }
    key[i] = kv;
  }
  __syncthreads();
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < n; i += 1024) {
        const int l = i ^ j;
        if (l > i) {
          const uint32_t x = key[i], y = key[l];
          if ((i & k) == 0 ? x > y : x < y) {
            key[i] = y;
            key[l] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  const int npairs = (nsub + 1) / 2;
  int32_t *out = map + bh * npairs * 2;
  for (int t = tid; t < 2 * npairs; t += 1024) out[t] = t < nsub ? (int32_t)(key[t] & 0xffffu) : nsub;
}

// ---------------------------------------------------------------------------
// 32-key score sub-tiles per 64-key stage, in every attention kernel.
constexpr int kStageSub = kBN / 32;

int launch_attn_dense(AttnArgs a, hipStream_t s) {
  constexpr int NW = 8;
  a.nqt = (a.Sq + 32 * NW - 1) / (32 * NW);
  const int64_t total = (int64_t)a.B * a.H * a.nqt;
  if (total > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "too many query tiles (%lld)", (long long)total);
  a.total = (int)total;
  hipLaunchKernelGGL((attn_fwd_pingpong_kernel<SwzLayout, kStageSub>), dim3(a.total), dim3(64 * NW), 0, s, a);
  return check_launch("attn_fwd_pingpong_kernel<dense>");
}

// Split-tail plan.  With one workgroup per CU, N whole 256-row tiles run in
// ceil(N / CUs) rounds and the last round keeps only N % CUs CUs busy (all of
// the chip idles but N for N < CUs).  Those r tiles are cut into P key
// ranges each, P = CUs / r (at least kMinSplitStages 64-key stages per
// range), so the last round is ~1/P as long.
static int device_cu_count(int *cus_out) {
  static std::atomic<int> cu_cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(H3A_ERR_HIP, "hipGetDevice failed");
  int cus = (dev >= 0 && dev < 64) ? cu_cache[dev].load(std::memory_order_relaxed) : 0;
  if (cus <= 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      return fail(H3A_ERR_HIP, "hipDeviceGetAttribute(multiProcessorCount) failed");
    if (dev >= 0 && dev < 64) cu_cache[dev].store(cus, std::memory_order_relaxed);
  }
  *cus_out = cus;
  return H3A_OK;
}

// `tiles` 256-row work items of up to `stages` stages each, split when
// `splittable`.  With `queued`, problems of at least kQueuedRounds rounds of
// tiles run on a persistent grid fed by the per-XCD queues (take_item): the
// XCDs' clocks differ under full load by up to ~5 %, and with a static
// deal the fastest XCD idles while the slowest finishes its share.
static int plan_tiles(int64_t tiles, int stages, bool splittable, bool queued, SplitPlan *plan) {
  constexpr int kMinSplitStages = 4;
  constexpr int64_t kQueuedRounds = 4;
  int cus = 0;
  const int rc = device_cu_count(&cus);
  if (rc) return rc;
  const int64_t r = tiles >= cus ? tiles % cus : tiles;
  int pieces = 1;
  if (splittable && r > 0) {
    const int64_t by_cus = cus / r, by_len = stages / kMinSplitStages;
    pieces = (int)(by_cus < by_len ? by_cus : by_len);
  }
  const int clamped = (int)(tiles > INT_MAX ? INT_MAX : tiles);
  *plan = SplitPlan{clamped, clamped, 1, 0, false, 0};
  if (tiles > INT_MAX) return H3A_OK;
  if (pieces >= 2) {
    plan->first = (int)(tiles - r);
    plan->pieces = pieces;
    plan->bytes = (size_t)r * pieces * 256 * (kD + 2) * sizeof(float);
  }
  if (queued && tiles >= kQueuedRounds * cus) {
    plan->dynamic = true;
    plan->sched_off = (plan->bytes + 255) & ~(size_t)255;
    plan->bytes = plan->sched_off + kSchedBytes;
  }
  return H3A_OK;
}

int plan_attn_split(int B, int H, int Sq, int Skv, SplitPlan *plan) {
  return plan_tiles((int64_t)B * H * ((Sq + 255) / 256), (Skv + kBN - 1) / kBN, true, true, plan);
}

// The longest list a query block can hold (max_k_blocks key blocks) stands in
// for the stage count.
int plan_attn_sparse_split(int B, int H, int Sq, int blk_q, int blk_k, int max_k_blocks, SplitPlan *plan) {
  const int rows = sparse_sub_block_rows(blk_q);
  const int64_t nsub = (Sq + rows - 1) / rows;
  return plan_tiles((int64_t)B * H * ((nsub + 1) / 2), max_k_blocks * (blk_k / 64), rows == 128, true, plan);
}

// The same for a tile LUT (64-row sub-blocks, unsplit): max_tiles entries
// stand in for the stage count.  The workspace starts with the pair map
// (tile_pair_map_kernel; up to kPairSortMax sub-blocks per (b,h), beyond
// that pairs 2p, 2p+1), then the queue counters.
int plan_attn_sparse_tiles(int B, int H, int Sq, int max_tiles, SplitPlan *plan) {
  const int64_t nsub = (Sq + 63) / 64;
  const int64_t pairs = (int64_t)B * H * ((nsub + 1) / 2);
  const int rc = plan_tiles(pairs, max_tiles, false, true, plan);
  if (rc || nsub > kPairSortMax || pairs > INT_MAX) return rc;
  const size_t map_bytes = (size_t)pairs * 2 * sizeof(int32_t);
  plan->pair_map = true;
  if (plan->dynamic) {
    plan->sched_off = (map_bytes + 255) & ~(size_t)255;
    plan->bytes = plan->sched_off + kSchedBytes;
  } else {
    plan->bytes = map_bytes;
  }
  return H3A_OK;
}

// Workgroups of a persistent launch of `kernel` (512 threads): every CU
// filled to its occupancy, cached per device.
// `slot` names the kernel in the cache (0 dense, 1 sparse pairs, 2 sparse
// key-split, 3 sparse key-split over tile masks).
static int persistent_grid(const void *kernel, int slot, int *grid) {
  static std::atomic<int> grid_cache[64][4];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(H3A_ERR_HIP, "hipGetDevice failed");
  std::atomic<int> *cached = (dev >= 0 && dev < 64) ? &grid_cache[dev][slot] : nullptr;
  int n = cached ? cached->load(std::memory_order_relaxed) : 0;
  if (n <= 0) {
    int cus = 0, per_cu = 0;
    const int rc = device_cu_count(&cus);
    if (rc) return rc;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 512, 0) != hipSuccess || per_cu <= 0)
      return fail(H3A_ERR_HIP, "hipOccupancyMaxActiveBlocksPerMultiprocessor failed");
    n = cus * per_cu;
    if (cached) cached->store(n, std::memory_order_relaxed);
  }
  *grid = n;
  return H3A_OK;
}

int launch_attn_dense_split(AttnArgs a, const SplitPlan &plan, void *ws, hipStream_t s) {
  if (plan.pieces < 2 && !plan.dynamic) return launch_attn_dense(a, s);
  a.nqt = (a.Sq + 255) / 256;
  if (plan.pieces >= 2) {
    a.split_first = plan.first;
    a.split_pieces = plan.pieces;
    a.ws = static_cast<float *>(ws);
  }
  const int64_t total = (int64_t)plan.first + (int64_t)(plan.tiles - plan.first) * plan.pieces;
  if (total > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "too many work items (%lld)", (long long)total);
  a.total = (int)total;
  auto kernel = attn_fwd_pingpong_kernel<SwzLayout, kStageSub>;
  int grid = a.total, rc;
  if (plan.dynamic) {
    rc = persistent_grid(reinterpret_cast<const void *>(kernel), 0, &grid);
    if (rc) return rc;
    if (grid > a.total) grid = a.total;
    a.sched = reinterpret_cast<int *>(static_cast<char *>(ws) + plan.sched_off);
    hipLaunchKernelGGL(sched_clear_kernel, dim3(1), dim3(256), 0, s, a.sched);
    rc = check_launch("sched_clear_kernel");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(512), 0, s, a);
  rc = check_launch("attn_fwd_pingpong_kernel<split>");
  if (rc || plan.pieces < 2) return rc;
  const int64_t rows = (int64_t)(plan.tiles - plan.first) * 256;
  hipLaunchKernelGGL(split_combine_kernel, dim3((unsigned)((rows + 7) / 8)), dim3(256), 0, s, a);
  return check_launch("split_combine_kernel");
}

// The block-sparse ping-pong kernel for query blocks of `rows` rows (with
// `tiles`: the key-split pairs over a tile LUT with sub-block masks); the
// wide-K/V instantiation when stage offsets from the (b,h) slice base could
// pass 2^32 bytes (see kWideKV).
typedef void (*PingPongKernel)(AttnArgs);
static PingPongKernel sparse_pingpong_kernel(const AttnArgs &a, int rows, bool tiles) {
  const int64_t stride = a.kss > a.vss ? a.kss : a.vss;
  const bool wide = ((int64_t)a.Skv + 64) * stride * 2 >= ((int64_t)1 << 32);
  if (tiles)
    return wide ? attn_fwd_pingpong_kernel<SwzLayout, kStageSub, true, true, true, true>
                : attn_fwd_pingpong_kernel<SwzLayout, kStageSub, true, true, false, true>;
  if (rows == 128)
    return wide ? attn_fwd_pingpong_kernel<SwzLayout, kStageSub, true, false, true>
                : attn_fwd_pingpong_kernel<SwzLayout, kStageSub, true, false, false>;
  return wide ? attn_fwd_pingpong_kernel<SwzLayout, kStageSub, true, true, true>
              : attn_fwd_pingpong_kernel<SwzLayout, kStageSub, true, true, false>;
}

int launch_attn_sparse_split(const AttnArgs &a, int blk_q, const SplitPlan &plan, void *ws, hipStream_t s,
                             bool tiles) {
  AttnArgs p = a;
  if (tiles && plan.pair_map) {
    int32_t *map = static_cast<int32_t *>(ws);
    hipLaunchKernelGGL(tile_pair_map_kernel, dim3((unsigned)(a.B * a.H)), dim3(1024), 0, s, a.counts, a.nqt,
                       a.lut_stride, map);
    const int rc = check_launch("tile_pair_map_kernel");
    if (rc) return rc;
    p.pair_map = map;
  }
  if (plan.pieces < 2 && !plan.dynamic) return launch_attn_sparse(p, blk_q, s, tiles);
  const int rows = tiles ? 64 : sparse_sub_block_rows(blk_q);
  if (plan.pieces >= 2 && rows != 128) return fail(H3A_ERR_INVALID_ARG, "split plan for 64-row query blocks");
  if (plan.pieces >= 2) {
    p.split_first = plan.first;
    p.split_pieces = plan.pieces;
    p.ws = static_cast<float *>(ws);
  }
  const int64_t total = (int64_t)plan.first + (int64_t)(plan.tiles - plan.first) * plan.pieces;
  if (total > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "too many work items (%lld)", (long long)total);
  p.total = (int)total;
  const PingPongKernel kernel = sparse_pingpong_kernel(p, rows, tiles);
  int grid = p.total, rc;
  if (plan.dynamic) {
    rc = persistent_grid(reinterpret_cast<const void *>(kernel), tiles ? 3 : (rows == 128 ? 1 : 2), &grid);
    if (rc) return rc;
    if (grid > p.total) grid = p.total;
    p.sched = reinterpret_cast<int *>(static_cast<char *>(ws) + plan.sched_off);
    hipLaunchKernelGGL(sched_clear_kernel, dim3(1), dim3(256), 0, s, p.sched);
    rc = check_launch("sched_clear_kernel");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(512), 0, s, p);
  rc = check_launch("attn_fwd_pingpong_kernel<sparse, split>");
  if (rc || plan.pieces < 2) return rc;
  const int64_t nrows = (int64_t)(plan.tiles - plan.first) * 256;
  hipLaunchKernelGGL(split_combine_kernel, dim3((unsigned)((nrows + 7) / 8)), dim3(256), 0, s, p);
  return check_launch("split_combine_kernel<sparse>");
}

int launch_attn_sparse(const AttnArgs &a, int blk_q, hipStream_t s, bool tiles) {
  const int rows = tiles ? 64 : sparse_sub_block_rows(blk_q);
  AttnArgs p = a;
  const int64_t pairs = (int64_t)a.B * a.H * ((a.nqt + 1) / 2);
  if (pairs > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "too many query-block pairs (%lld)", (long long)pairs);
  p.total = (int)pairs;
  hipLaunchKernelGGL(sparse_pingpong_kernel(p, rows, tiles), dim3(p.total), dim3(512), 0, s, p);
  return check_launch("attn_fwd_pingpong_kernel<sparse>");
}

int launch_block_map_to_lut(const uint8_t *map, int B, int H, int nq, int nk, int32_t *lut,
                            int32_t *counts, int max_k_blocks, hipStream_t s) {
  const int64_t rows = (int64_t)B * H * nq;
  const int64_t blocks = (rows + 255) / 256;
  hipLaunchKernelGGL(block_map_to_lut_kernel, dim3((unsigned)blocks), dim3(256), 0, s, map, rows, nk,
                     lut, counts, max_k_blocks);
  return check_launch("block_map_to_lut_kernel");
}

int launch_test_qk(const uint16_t *Q, const uint16_t *K, float *S, hipStream_t s) {
  hipLaunchKernelGGL(test_qk_kernel, dim3(1), dim3(64), 0, s, Q, K, S);
  return check_launch("test_qk_kernel");
}

int launch_test_pv(const uint16_t *P, const uint16_t *V, float *O, hipStream_t s) {
  hipLaunchKernelGGL(test_pv_kernel, dim3(1), dim3(64), 0, s, P, V, O);
  return check_launch("test_pv_kernel");
}

static int fill_attrs(const void *fn, int threads, double out[6]) {
  hipFuncAttributes fa;
  if (hipFuncGetAttributes(&fa, fn) != hipSuccess) return fail(H3A_ERR_HIP, "hipFuncGetAttributes failed");
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, threads, 0) != hipSuccess)
    return fail(H3A_ERR_HIP, "hipOccupancyMaxActiveBlocksPerMultiprocessor failed");
  int dev = 0, clk = 0, max_threads = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&clk, hipDeviceAttributeClockRate, dev) != hipSuccess ||
      hipDeviceGetAttribute(&max_threads, hipDeviceAttributeMaxThreadsPerMultiProcessor, dev) != hipSuccess)
    return fail(H3A_ERR_HIP, "hipDeviceGetAttribute failed");
  out[0] = fa.numRegs;
  out[1] = (double)fa.sharedSizeBytes;
  out[2] = blocks;
  out[3] = clk;
  out[4] = max_threads > 0 ? (double)(blocks * threads) / max_threads : 0.0;
  out[5] = threads;
  return H3A_OK;
}

// Phase profile readout (profile build; zeros otherwise).  Synchronises the
// device first, as the reference's cudaMemcpyFromSymbol did implicitly.
int attn_prof_read(uint64_t *out) {
  if (hipDeviceSynchronize() != hipSuccess) return fail(H3A_ERR_HIP, "hipDeviceSynchronize failed");
  if (hipMemcpyFromSymbol(out, HIP_SYMBOL(g_prof), sizeof(g_prof), 0, hipMemcpyDeviceToHost) != hipSuccess)
    return fail(H3A_ERR_HIP, "hipMemcpyFromSymbol(g_prof) failed");
  return H3A_OK;
}

int attn_prof_reset() {
  static const unsigned long long zeros[H3A_PROF_WAVES][kProfSlots] = {};
  if (hipDeviceSynchronize() != hipSuccess) return fail(H3A_ERR_HIP, "hipDeviceSynchronize failed");
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_prof), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice) != hipSuccess)
    return fail(H3A_ERR_HIP, "hipMemcpyToSymbol(g_prof) failed");
  return H3A_OK;
}

int attn_kernel_attrs(int which, double out[6]) {
  switch (which) {
    case H3A_KERNEL_ATTN_DENSE:
      return fill_attrs(reinterpret_cast<const void *>(&attn_fwd_pingpong_kernel<SwzLayout, kStageSub>), 512, out);
    case H3A_KERNEL_ATTN_SPARSE_128:
      return fill_attrs(reinterpret_cast<const void *>(&attn_fwd_pingpong_kernel<SwzLayout, kStageSub, true>), 512,
                        out);
    case H3A_KERNEL_ATTN_SPARSE_64:
      return fill_attrs(reinterpret_cast<const void *>(&attn_fwd_pingpong_kernel<SwzLayout, kStageSub, true, true>),
                        512, out);
    case H3A_KERNEL_ATTN_SPARSE_TILES:
      return fill_attrs(
          reinterpret_cast<const void *>(&attn_fwd_pingpong_kernel<SwzLayout, kStageSub, true, true, false, true>),
          512, out);
    default:
      return fail(H3A_ERR_INVALID_ARG, "unknown kernel id %d", which);
  }
}

}  // namespace h3a
