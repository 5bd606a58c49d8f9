// Block-map construction for the block-sparse (h3_sla) path, on the GPU.
//
// The reference gets its block map from SLA's get_block_map
// (custom_nodes/h3_sla/__init__.py:232): mean-pool q and k over blocks of
// rows, score every (query block, key block) pair by the dot product of the
// pooled vectors, keep the top-k key blocks of each query block.  Here:
//   block_pool_kernel   : bf16 [B,H,S,128] (strided) -> fp32 block means
//                         [B,H,ceil(S/blk),128], over the valid rows of each
//                         block.  HBM-bound: reads the tensor once.
//   block_select_kernel : up to 16 query blocks of one (b,h) per workgroup:
//                         scores against all key blocks (fp32 MFMA) into LDS, rank by
//                         (score desc, index asc), keep rank < keep plus the
//                         optional diagonal, and write the kept indices in
//                         ascending order (the LUT h3a_attn_fwd_blocksparse
//                         consumes), the count, and optionally the 0/1 map.
// Centring k by its sequence mean (SLA's K smoothing) shifts every score of a
// row by the same amount, so it never changes the selection and is not needed.
#include <type_traits>

#include "h3a_device.h"
#include "h3a_internal.h"
#include "h3a_queue.h"

namespace h3a {

constexpr int kPoolD = 128;

// One wave per (b,h,block): lane = 16*rg + c holds dims 8c..8c+7 of rows rg, rg+4, ...
__global__ void __launch_bounds__(256) block_pool_kernel(const uint16_t *x, int64_t sb, int64_t sh,
                                                         int64_t ss, int H, int S, int blk, int nb,
                                                         int64_t items, float *out) {
  const int tid = threadIdx.x, lane = tid & 63, rg = lane >> 4, c = lane & 15;
  const int64_t item = (int64_t)blockIdx.x * 4 + (tid >> 6);
  if (item >= items) return;  // whole waves leave together
  const int j = (int)(item % nb);
  const int64_t bh = item / nb;
  const int h = (int)(bh % H), b = (int)(bh / H);
  const int r0 = j * blk;
  const int rows = (S - r0) < blk ? (S - r0) : blk;
  const uint16_t *base = x + b * sb + h * sh + (int64_t)r0 * ss + c * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int r = rg; r < rows; r += 4) {
    const u32x4 w = *(const u32x4 *)(base + (int64_t)r * ss);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += bf16_lo(w[i]);
      acc[2 * i + 1] += bf16_hi(w[i]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    acc[e] += __shfl_xor(acc[e], 16);
    acc[e] += __shfl_xor(acc[e], 32);
  }
  if (rg == 0) {
    const float inv = 1.f / (float)rows;
    float *o = out + item * kPoolD + c * 8;
#pragma unroll
    for (int e = 0; e < 8; e += 4)
      *(float4 *)(o + e) = float4{acc[e] * inv, acc[e + 1] * inv, acc[e + 2] * inv, acc[e + 3] * inv};
  }
}

constexpr int kSelThreads = 256;
constexpr int kSelRowsPerWave = 4;
constexpr int kSelRowsMax = kSelRowsPerWave * (kSelThreads / 64);  // query blocks per workgroup
// Rows of up to 768 key blocks (12 chunks of 64) and of more than 3072 run in
// 4-wave workgroups whose dynamic LDS caps the score rows (R rows of nk floats,
// plus one spare float) at 40 KiB, so that four workgroups fit on a CU: 16
// rows up to nk = 639, 15 at 659, 3 at 3073, 1 at the 7000 maximum.
constexpr int kSelScoreBytes = 40960 - 4;
// Rows of 769 to 1536 key blocks (13 to 24 chunks) run in 8-wave workgroups,
// two per CU, over 80,000 bytes of static LDS each (16 rows up to nk = 1249,
// 15 at 1317, 13 at 1536), two rows per wave in registers; rows of 1537 to
// 3072 (25 to 48 chunks) in one 16-wave workgroup per CU over 160,000 bytes
// (16 rows up to nk = 2499, 15 at 2633, 13 at 3072), one row per wave.  The
// head's pooled keys are then read once per 13-16 rows instead of once per
// 3-8; two workgroups per CU where they fit, so that one workgroup's score
// phase overlaps another's selection.
constexpr int kSelMidWaves = 8;
constexpr int kSelMidScoreFloats = 20000;
constexpr int kSelWideWaves = 16;
constexpr int kSelWideScoreFloats = 40000;
constexpr int kSelKeyTile = 16;  // key blocks per score tile (one MFMA output tile)

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Dims of step m = 4j + t of the score MFMAs, for k-slot s (lane / 16):
// 16j + 4s + t, so each lane's operands for steps 4j..4j+3 are one 16-byte
// load and the 32 steps cover d = 0..127 once.
__device__ __forceinline__ void load_score_operand(f32x4 (&x)[8], const float *row, int slot) {
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = *(const f32x4 *)(row + 16 * j + 4 * slot);
}

// R (<= kSelRowsMax = 16) query blocks of one (b,h) per workgroup of NW
// waves, so each pooled key vector is read from memory once per R rows.
// Scores: the 16 rows x 16 key blocks of a tile are one chain of 32
// v_mfma_f32_16x16x4f32 (fp32 products and sums); wave w takes key tiles w,
// w+NW, ..., its pooled keys loaded straight into registers one tile ahead,
// and writes the tile's scores to LDS.  Then wave
// w selects rows w, w+NW, ..., with lane l on key blocks j = 64c + l: a bitwise
// search over order-preserving keys finds the row's keep-th largest score in
// 32 counting rounds (ballot + popcount), which fixes the kept set under
// (score desc, index asc) order without ranking every pair.  Kept indices are
// written in ascending order with one ballot per 64-key chunk.
template <int NW>
__global__ void __launch_bounds__(NW * 64, NW == kSelMidWaves ? 4 : 1) block_select_kernel(
    const float *pq, const float *pk, int nq, int nk, int rows_per_wg, int keep, int force_diag,
    int blk_q, int blk_k, int32_t *lut, int32_t *counts, int max_k, uint8_t *map) {
  static_assert(NW == kSelThreads / 64 || NW == kSelMidWaves || NW == kSelWideWaves, "4, 8 or 16 waves");
  // [R][nk] scores, then one spare slot: dynamic LDS (4 waves), or static
  // LDS sized for the longest rows of the 16-wave form.
  float *sc;
  if constexpr (NW == kSelWideWaves) {
    __shared__ float sc_wide[kSelWideScoreFloats];
    sc = sc_wide;
  } else if constexpr (NW == kSelMidWaves) {
    __shared__ float sc_mid[kSelMidScoreFloats];
    sc = sc_mid;
  } else {
    extern __shared__ float sc_dyn[];
    sc = sc_dyn;
  }
  // The wave index as a scalar, so the loops over a wave's tiles and rows are uniform.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int R = rows_per_wg;
  const int ngroups = (nq + R - 1) / R;
  // Consecutive row groups (those of one head) run on one XCD, so that head's
  // pooled keys come from that XCD's L2 after the first group reads them.
  const int g = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int64_t bh = g / ngroups;
  const int i0 = (g % ngroups) * R;
  const int nrows = nq - i0 < R ? nq - i0 : R;
  // MFMA operands: lane l supplies A[row l%16][slot l/16] (query rows, past
  // nrows clamped to the last one; their scores are not stored) and
  // B[slot l/16][key l%16]; lane l's results are rows 4*(l/16) + v, v = 0..3,
  // of key l%16.
  static_assert(kSelRowsMax == 16, "one MFMA tile spans the workgroup's rows");
  const int lr = lane & 15, slot = lane >> 4;
  f32x4 qa[8];
  load_score_operand(qa, pq + (bh * nq + i0 + (lr < nrows ? lr : nrows - 1)) * kPoolD, slot);
  const float *pkh = pk + bh * (int64_t)nk * kPoolD;
  const int ntiles = (nk + kSelKeyTile - 1) / kSelKeyTile;
  // Key rows past nk repeat the last key block (the tile after a wave's last
  // one too); their scores are not stored.
  auto key_row = [&](int t) __attribute__((always_inline)) {
    const int j = t * kSelKeyTile + lr;
    return pkh + (int64_t)(j < nk ? j : nk - 1) * kPoolD;
  };
  auto score_tile = [&](int t, const f32x4(&kb)[8]) __attribute__((always_inline)) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[j][u], kb[j][u], acc, 0, 0, 0);
    // Scores of rows past nrows or keys past nk go to the spare slot sc[R*nk]
    // (no branches around the stores).
    const int key = t * kSelKeyTile + lr;
#pragma unroll
    for (int v = 0; v < 4; ++v)
      sc[4 * slot + v < nrows && key < nk ? (4 * slot + v) * nk + key : R * nk] = acc[v];
  };
  // Two key buffers, each loaded while the other one's tile is scored (the
  // scheduling barriers keep the loads ahead of the MFMA chain they overlap).
  f32x4 k0[8], k1[8];
  load_score_operand(k0, key_row(wave < ntiles ? wave : ntiles - 1), slot);
  for (int t = wave; t < ntiles; t += 2 * NW) {
    load_score_operand(k1, key_row(t + NW < ntiles ? t + NW : ntiles - 1), slot);
    __builtin_amdgcn_sched_barrier(0);
    score_tile(t, k0);
    load_score_operand(k0, key_row(t + 2 * NW < ntiles ? t + 2 * NW : ntiles - 1), slot);
    __builtin_amdgcn_sched_barrier(0);
    if (t + NW < ntiles) score_tile(t + NW, k1);
  }
  __syncthreads();

  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));  // lanes < this one
  // Order-preserving key of a score: larger score <=> larger key (-0 as +0).
  auto key_of = [](float x) __attribute__((always_inline)) -> uint32_t {
    const uint32_t u = __float_as_uint(x + 0.f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  };
  const int nchunks = (nk + 63) / 64;
  // Kept set of row r from its threshold: exactly the keys > T and the first
  // `need` keys == T in index order (rank < keep under (score desc, index
  // asc)), plus the optional diagonal; indices written in ascending order.
  auto write_row = [&](int r, uint32_t T, int need) __attribute__((always_inline)) {
    const float *row_sc = sc + r * nk;
    const int64_t row = bh * nq + i0 + r;
    const int diag = (int)(((int64_t)(i0 + r) * blk_q) / blk_k);
    int32_t *out = lut + row * max_k;
    int base = 0, eq_before = 0;
    for (int c = 0; c < nchunks; ++c) {
      const int j = c * 64 + lane;
      const uint32_t kj = j < nk ? key_of(row_sc[j < nk ? j : 0]) : 0u;
      const bool eq = keep > 0 && j < nk && kj == T;
      const uint64_t eqm = __builtin_amdgcn_ballot_w64(eq);
      const bool by_rank = keep > 0 && j < nk && (kj > T || (eq && eq_before + __builtin_popcountll(eqm & below) < need));
      const bool kept = by_rank || (force_diag && j == diag && j < nk);
      eq_before += __builtin_popcountll(eqm);
      const uint64_t m = __builtin_amdgcn_ballot_w64(kept);
      const int pos = base + __builtin_popcountll(m & below);
      if (kept && pos < max_k) out[pos] = j;
      if (map && j < nk) map[row * nk + j] = (uint8_t)kept;
      base += __builtin_popcountll(m);
    }
    const int kept_n = base < max_k ? base : max_k;
    for (int t = kept_n + lane; t < max_k; t += 64) out[t] = -1;
    if (lane == 0) counts[row] = kept_n;
  };
  // T = the keep-th largest key of a row: the largest t with (number of the
  // row's keys >= t) >= keep, built from the top bit down; need = keep - the
  // number of keys > T.  Every t asked for is >= 1, every score that is not a
  // NaN has a key > 0, and the padding key 0 is never counted.  The search
  // stops early once exactly keep keys are >= the candidate c: the kept set
  // is then {keys >= c}, written as T = c - 1, need = 0.
  //
  // Rows of up to NC*64 key blocks: the keys of all of this wave's rows
  // (wave + NW*i, i < RPW) sit in registers, NC per lane per row, and the
  // rows' searches run interleaved, so their 32 dependent counting rounds
  // overlap.  (NC, RPW) = (6, 4) or (12, 4) with 4 waves, (24, 2) with 8,
  // (48, 1) with 16: at most 48 registers of keys, for 16 rows.
  auto select_rows_regs = [&](auto nc_const, auto rpw_const) __attribute__((always_inline)) {
    constexpr int NC = decltype(nc_const)::value;
    constexpr int RPW = decltype(rpw_const)::value;
    uint32_t T[RPW], kr[RPW][NC];
    int need[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int r = wave + NW * i;
      const float *row_sc = sc + (r < nrows ? r : 0) * nk;
      T[i] = 0;
      need[i] = 0;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int j = c * 64 + lane;
        kr[i][c] = (r < nrows && j < nk) ? key_of(row_sc[j < nk ? j : 0]) : 0u;
      }
    }
    auto count_ge = [&](const uint32_t(&k)[NC], uint32_t t) __attribute__((always_inline)) -> int {
      int n = 0;
#pragma unroll
      for (int c = 0; c < NC; ++c) n += __builtin_popcountll(__builtin_amdgcn_ballot_w64(k[c] >= t));
      return n;
    };
    if (keep > 0) {
      bool done[RPW];
#pragma unroll
      for (int i = 0; i < RPW; ++i) done[i] = wave + NW * i >= nrows;
      for (int bit = 31; bit >= 0; --bit) {
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
          if (done[i]) continue;
          const uint32_t cand = T[i] | (1u << bit);
          const int n = count_ge(kr[i], cand);
          if (n >= keep) T[i] = cand;
          if (n == keep) {
            T[i] = cand - 1;
            done[i] = true;
          }
        }
        bool all = true;
#pragma unroll
        for (int i = 0; i < RPW; ++i) all = all && done[i];
        if (all) break;
      }
#pragma unroll
      for (int i = 0; i < RPW; ++i)
        need[i] = done[i] ? 0 : keep - (T[i] == 0xffffffffu ? 0 : count_ge(kr[i], T[i] + 1));
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i)
      if (wave + NW * i < nrows) write_row(wave + NW * i, T[i], need[i]);
  };
  // Longer rows: one row at a time, keys re-read from LDS every round.
  auto select_rows_lds = [&]() __attribute__((always_inline)) {
    for (int r = wave; r < nrows; r += NW) {
      const float *row_sc = sc + r * nk;
      auto count_ge = [&](uint32_t t) __attribute__((always_inline)) -> int {
        int n = 0;
        for (int c = 0; c < nchunks; ++c) {
          const int j = c * 64 + lane;
          n += __builtin_popcountll(__builtin_amdgcn_ballot_w64(j < nk && key_of(row_sc[j < nk ? j : 0]) >= t));
        }
        return n;
      };
      uint32_t T = 0;
      int need = 0;
      if (keep > 0) {
        bool done = false;
        for (int bit = 31; bit >= 0 && !done; --bit) {
          const uint32_t cand = T | (1u << bit);
          const int n = count_ge(cand);
          if (n >= keep) T = cand;
          if (n == keep) {
            T = cand - 1;
            done = true;
          }
        }
        if (!done) need = keep - (T == 0xffffffffu ? 0 : count_ge(T + 1));
      }
      write_row(r, T, need);
    }
  };
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  if constexpr (NW == kSelMidWaves) {
    if (nchunks <= 24 && nrows <= 2 * NW)
      select_rows_regs(std::integral_constant<int, 24>{}, I2{});
    else
      select_rows_lds();
  } else if constexpr (NW == kSelWideWaves) {
    if (nchunks <= 48 && nrows <= NW)
      select_rows_regs(std::integral_constant<int, 48>{}, I1{});
    else
      select_rows_lds();
  } else {
    if (nchunks <= 6)
      select_rows_regs(std::integral_constant<int, 6>{}, I4{});
    else if (nchunks <= 12)
      select_rows_regs(std::integral_constant<int, 12>{}, I4{});
    else
      select_rows_lds();
  }
}

// ---------------------------------------------------------------------------
// Tile LUTs, for block sizes the native block-sparse kernels do not take (any
// multiple of 16, in either dimension).  The attention then runs on 64-row
// query sub-blocks; the tile LUT row of sub-block qs lists, ascending, every
// 32-key column holding a kept (query block, key block) pair for some row of
// qs, as column << 8 | mask.  Bit 2*i + j of the mask is set when rows
// 64*qs + 16*i .. +15 and keys 32*column + 16*j .. +15 lie in a kept pair;
// both block sizes are multiples of 16, so each 16x16 sub-block lies in
// exactly one pair.  Sub-blocks past Sq or Skv get no bit.  One wave per LUT
// row; lane l takes columns 64*c + l, and the kept ones are written in order
// with one ballot per 64 columns.  Entries past the count are -1.
__global__ void __launch_bounds__(256) block_map_to_tile_lut_kernel(const uint8_t *map, int64_t rows, int nsub,
                                                                    int nq, int nk, int Sq, int Skv, int blk_q,
                                                                    int blk_k, int ncols, int32_t *lut,
                                                                    int32_t *counts, int max_tiles) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves leave together
  const int qs = (int)(row % nsub);
  const int64_t bh = row / nsub;
  // Map row of each 16-row slice of the sub-block (null past Sq).
  const uint8_t *mq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 64 * qs + 16 * i;
    mq[i] = r < Sq ? map + (bh * nq + r / blk_q) * (int64_t)nk : nullptr;
  }
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int32_t *out = lut + row * (int64_t)max_tiles;
  int base = 0;
  for (int c = 0; c < ncols; c += 64) {
    const int col = c + lane;
    uint32_t mask = 0;
    if (col < ncols) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int key = 32 * col + 16 * j;
        if (key >= Skv) break;
        const int kb = key / blk_k;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (mq[i] && mq[i][kb]) mask |= 1u << (2 * i + j);
      }
    }
    const uint64_t m = __builtin_amdgcn_ballot_w64(mask != 0);
    const int pos = base + __builtin_popcountll(m & below);
    if (mask != 0 && pos < max_tiles) out[pos] = (int32_t)(((uint32_t)col << 8) | mask);
    base += __builtin_popcountll(m);
  }
  const int kept = base < max_tiles ? base : max_tiles;
  for (int j = kept + lane; j < max_tiles; j += 64) out[j] = -1;
  if (lane == 0) counts[row] = kept;
}

// A block LUT -> 0/1 block map [rows, nk]: the map is cleared by one launch,
// and the next sets the listed blocks (entries outside [0, nk), and those past
// a row's count, are ignored).  Two launches, so that no byte is written by
// two threads of one kernel.
__global__ void __launch_bounds__(256) clear_bytes_kernel(uint8_t *p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}

__global__ void __launch_bounds__(256) lut_scatter_kernel(const int32_t *lut, const int32_t *counts, int64_t rows,
                                                          int nk, int max_k, uint8_t *map) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int cnt = counts[row];
  const int n = cnt < 0 ? 0 : (cnt > max_k ? max_k : cnt);
  for (int e = lane; e < n; e += 64) {
    const int kb = lut[row * (int64_t)max_k + e];
    if (kb >= 0 && kb < nk) map[row * (int64_t)nk + kb] = 1;
  }
}

int launch_block_map_to_tile_lut(const uint8_t *map, int B, int H, int Sq, int Skv, int blk_q, int blk_k,
                                 int32_t *lut, int32_t *counts, int max_tiles, hipStream_t s) {
  const int nsub = (Sq + 63) / 64, nq = (Sq + blk_q - 1) / blk_q, nk = (Skv + blk_k - 1) / blk_k;
  const int ncols = (Skv + 31) / 32;
  const int64_t rows = (int64_t)B * H * nsub;
  hipLaunchKernelGGL(block_map_to_tile_lut_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, map, rows,
                     nsub, nq, nk, Sq, Skv, blk_q, blk_k, ncols, lut, counts, max_tiles);
  return check_launch("block_map_to_tile_lut_kernel");
}

int launch_lut_to_block_map(const int32_t *lut, const int32_t *counts, int B, int H, int nq, int nk,
                            int max_k_blocks, uint8_t *map, hipStream_t s) {
  const int64_t rows = (int64_t)B * H * nq, bytes = rows * nk;
  const int64_t clear_blocks = (bytes + 255) / 256 < 65536 ? (bytes + 255) / 256 : 65536;
  hipLaunchKernelGGL(clear_bytes_kernel, dim3((unsigned)clear_blocks), dim3(256), 0, s, map, bytes);
  int rc = check_launch("clear_bytes_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(lut_scatter_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, lut, counts, rows, nk,
                     max_k_blocks, map);
  return check_launch("lut_scatter_kernel");
}

int launch_block_pool(const uint16_t *x, const int64_t st[3], int B, int H, int S, int blk,
                      float *out, hipStream_t s) {
  const int nb = (S + blk - 1) / blk;
  const int64_t items = (int64_t)B * H * nb;
  hipLaunchKernelGGL(block_pool_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, x, st[0],
                     st[1], st[2], H, S, blk, nb, items, out);
  return check_launch("block_pool_kernel");
}

int launch_block_select(const float *pq, const float *pk, int B, int H, int nq, int nk, int keep,
                        int force_diag, int blk_q, int blk_k, int32_t *lut, int32_t *counts,
                        int max_k, uint8_t *map, hipStream_t s) {
  const int nchunks = (nk + 63) / 64;
  if (nchunks > 12 && nchunks <= 24) {
    int rows = (kSelMidScoreFloats - 1) / nk;
    rows = rows > kSelRowsMax ? kSelRowsMax : rows;  // >= 13 for nk <= 1536
    const int64_t groups = (int64_t)B * H * ((nq + rows - 1) / rows);
    hipLaunchKernelGGL(block_select_kernel<kSelMidWaves>, dim3((unsigned)groups), dim3(kSelMidWaves * 64), 0,
                       s, pq, pk, nq, nk, rows, keep, force_diag, blk_q, blk_k, lut, counts, max_k, map);
    return check_launch("block_select_kernel<8 waves>");
  }
  if (nchunks > 24 && nchunks <= 48) {
    int rows = (kSelWideScoreFloats - 1) / nk;
    rows = rows > kSelRowsMax ? kSelRowsMax : rows;  // >= 13 for nk <= 3072
    const int64_t groups = (int64_t)B * H * ((nq + rows - 1) / rows);
    hipLaunchKernelGGL(block_select_kernel<kSelWideWaves>, dim3((unsigned)groups), dim3(kSelWideWaves * 64), 0,
                       s, pq, pk, nq, nk, rows, keep, force_diag, blk_q, blk_k, lut, counts, max_k, map);
    return check_launch("block_select_kernel<16 waves>");
  }
  int rows = kSelScoreBytes / (nk * (int)sizeof(float));
  rows = rows < 1 ? 1 : (rows > kSelRowsMax ? kSelRowsMax : rows);
  const size_t lds = ((size_t)rows * nk + 1) * sizeof(float);
  const int64_t groups = (int64_t)B * H * ((nq + rows - 1) / rows);
  hipLaunchKernelGGL(block_select_kernel<kSelThreads / 64>, dim3((unsigned)groups), dim3(kSelThreads), lds, s,
                     pq, pk, nq, nk, rows, keep, force_diag, blk_q, blk_k, lut, counts, max_k, map);
  return check_launch("block_select_kernel");
}

}  // namespace h3a
