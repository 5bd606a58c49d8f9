// Block-map construction for the block-sparse (h3_sla) path, on the GPU.
//
// The reference gets its block map from SLA's get_block_map
// (custom_nodes/h3_sla/__init__.py:232): mean-pool q and k over blocks of
// rows, score every (query block, key block) pair by the dot product of the
// pooled vectors, keep the top-k key blocks of each query block.  Here:
//   block_pool_kernel   : bf16 [B,H,S,128] (strided) -> fp32 block means
//                         [B,H,ceil(S/blk),128], over the valid rows of each
//                         block.  HBM-bound: reads the tensor once.
//   block_select_kernel : up to 8 query blocks of one (b,h) per workgroup:
//                         scores against all key blocks into LDS, rank by
//                         (score desc, index asc), keep rank < keep plus the
//                         optional diagonal, and write the kept indices in
//                         ascending order (the LUT h3a_attn_fwd_blocksparse
//                         consumes), the count, and optionally the 0/1 map.
// Centring k by its sequence mean (SLA's K smoothing) shifts every score of a
// row by the same amount, so it never changes the selection and is not needed.
#include <type_traits>

#include "h3a_device.h"
#include "h3a_internal.h"

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
#ifndef H3A_SEL_ROWS
#define H3A_SEL_ROWS 8
#endif
constexpr int kSelRowsMax = H3A_SEL_ROWS;  // query blocks per workgroup (at most)
constexpr int kSelKeyChunk = 32;        // pooled key vectors staged in LDS at a time
constexpr int kSelKeyPitch = kPoolD + 4; // floats per staged key row (bank spread)
// LDS for the score rows: 64 KiB minus the query rows and the key chunk.
constexpr int kSelScoreBytes = 65536 - (H3A_SEL_ROWS * kPoolD + kSelKeyChunk * kSelKeyPitch) * 4;

// R (<= kSelRowsMax) query blocks of one (b,h) per workgroup, so each pooled
// key vector is read from memory once per R rows.  Scores of all R rows go to
// LDS (same fp32 FMA order as a plain dot product over d = 0..127).  Then wave
// w selects rows w, w+4, with lane l on key blocks j = 64c + l: a bitwise
// search over order-preserving keys finds the row's keep-th largest score in
// 32 counting rounds (ballot + popcount), which fixes the kept set under
// (score desc, index asc) order without ranking every pair.  Kept indices are
// written in ascending order with one ballot per 64-key chunk.
__global__ void __launch_bounds__(kSelThreads) block_select_kernel(
    const float *pq, const float *pk, int nq, int nk, int rows_per_wg, int keep, int force_diag,
    int blk_q, int blk_k, int32_t *lut, int32_t *counts, int max_k, uint8_t *map) {
  extern __shared__ float sel_lds[];
  float *qs = sel_lds;                                   // [kSelRowsMax][128] pooled query blocks
  float *ks = qs + kSelRowsMax * kPoolD;                 // [kSelKeyChunk][kSelKeyPitch] key chunk
  float *sc = ks + kSelKeyChunk * kSelKeyPitch;          // [R][nk] scores
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int R = rows_per_wg;
  const int ngroups = (nq + R - 1) / R;
  const int64_t bh = blockIdx.x / ngroups;
  const int i0 = (int)(blockIdx.x % ngroups) * R;
  const int nrows = nq - i0 < R ? nq - i0 : R;
  for (int t = tid; t < kSelRowsMax * kPoolD; t += kSelThreads) {
    const int r = t / kPoolD;
    qs[t] = r < nrows ? pq[((bh * nq) + i0 + r) * kPoolD + (t % kPoolD)] : 0.f;
  }
  // Scores, kSelKeyChunk key blocks at a time: the chunk is staged with
  // coalesced 16-byte loads, then thread (r, kk) forms one dot product in
  // the order d = 0..127.
  const float *pkh = pk + bh * (int64_t)nk * kPoolD;
  const int my_r = tid / kSelKeyChunk, my_k = tid % kSelKeyChunk;
  static_assert(kSelRowsMax * kSelKeyChunk <= kSelThreads, "one dot product per thread per chunk");
  for (int kc = 0; kc < nk; kc += kSelKeyChunk) {
    __syncthreads();  // qs written / previous chunk consumed
    for (int t = tid; t < kSelKeyChunk * (kPoolD / 4); t += kSelThreads) {
      const int kk = t / (kPoolD / 4), f4 = t % (kPoolD / 4);
      const float4 v = kc + kk < nk ? *(const float4 *)(pkh + (int64_t)(kc + kk) * kPoolD + 4 * f4)
                                    : float4{0.f, 0.f, 0.f, 0.f};
      *(float4 *)(ks + kk * kSelKeyPitch + 4 * f4) = v;
    }
    __syncthreads();
    if (my_r < nrows && kc + my_k < nk) {
      const float *qr = qs + my_r * kPoolD;
      const float *kr = ks + my_k * kSelKeyPitch;
      float acc = 0.f;
#pragma unroll 8
      for (int d = 0; d < kPoolD; d += 4) {
        const float4 q4 = *(const float4 *)(qr + d);
        const float4 k4 = *(const float4 *)(kr + d);
        acc = fmaf(q4.x, k4.x, acc);
        acc = fmaf(q4.y, k4.y, acc);
        acc = fmaf(q4.z, k4.z, acc);
        acc = fmaf(q4.w, k4.w, acc);
      }
      sc[my_r * nk + kc + my_k] = acc;
    }
  }
  __syncthreads();

  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));  // lanes < this one
  // Order-preserving key of a score: larger score <=> larger key (-0 as +0).
  auto key_of = [](float x) __attribute__((always_inline)) -> uint32_t {
    const uint32_t u = __float_as_uint(x + 0.f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  };
  const int nchunks = (nk + 63) / 64;
  // NC > 0: the row's keys are held in NC registers per lane for the counting
  // rounds (rows of up to NC*64 key blocks); NC = 0: longer rows re-read
  // them from LDS each round.
  auto select_rows = [&](auto nc_const) __attribute__((always_inline)) {
    constexpr int NC = decltype(nc_const)::value;
    constexpr int kSelRegChunks = NC > 0 ? NC : 1;
    constexpr bool in_regs = NC > 0;
    for (int r = wave; r < nrows; r += kSelThreads / 64) {
      const float *row_sc = sc + r * nk;
      const int64_t row = bh * nq + i0 + r;
      const int diag = (int)(((int64_t)(i0 + r) * blk_q) / blk_k);
      int32_t *out = lut + row * max_k;
      uint32_t kr[kSelRegChunks];  // valid keys; 0 (never counted: t >= 1 below) past nk
#pragma unroll
      for (int c = 0; c < kSelRegChunks; ++c) {
        const int j = c * 64 + lane;
        kr[c] = (in_regs && j < nk) ? key_of(row_sc[j < nk ? j : 0]) : 0u;
      }
      // Number of the row's keys >= t.  Every t asked for is >= 1, every score
      // that is not a NaN has a key > 0, and the padding key 0 is never counted.
      auto count_ge = [&](uint32_t t) __attribute__((always_inline)) -> int {
        int n = 0;
        if constexpr (in_regs) {
#pragma unroll
          for (int c = 0; c < kSelRegChunks; ++c) n += __builtin_popcountll(__builtin_amdgcn_ballot_w64(kr[c] >= t));
        } else {
          for (int c = 0; c < nchunks; ++c) {
            const int j = c * 64 + lane;
            n += __builtin_popcountll(__builtin_amdgcn_ballot_w64(j < nk && key_of(row_sc[j < nk ? j : 0]) >= t));
          }
        }
        return n;
      };
      // T = the keep-th largest key: the largest t with count_ge(t) >= keep,
      // built from the top bit down.  Then exactly the keys > T and the first
      // (keep - #keys > T) keys == T in index order have rank < keep under
      // (score desc, index asc).
      uint32_t T = 0;
      int need = 0;  // keys == T to keep
      if (keep > 0) {
        for (int bit = 31; bit >= 0; --bit) {
          const uint32_t cand = T | (1u << bit);
          if (count_ge(cand) >= keep) T = cand;
        }
        need = keep - (T == 0xffffffffu ? 0 : count_ge(T + 1));
      }
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
    }
  };
  if (nchunks <= 6)
    select_rows(std::integral_constant<int, 6>{});
  else if (nchunks <= 12)
    select_rows(std::integral_constant<int, 12>{});
  else
    select_rows(std::integral_constant<int, 0>{});
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
  int rows = kSelScoreBytes / (nk * (int)sizeof(float));
  rows = rows < 1 ? 1 : (rows > kSelRowsMax ? kSelRowsMax : rows);
  const size_t lds = (size_t)(kSelRowsMax * kPoolD + kSelKeyChunk * kSelKeyPitch + rows * nk) * sizeof(float);
  const int64_t groups = (int64_t)B * H * ((nq + rows - 1) / rows);
  hipLaunchKernelGGL(block_select_kernel, dim3((unsigned)groups), dim3(kSelThreads), lds, s, pq, pk, nq,
                     nk, rows, keep, force_diag, blk_q, blk_k, lut, counts, max_k, map);
  return check_launch("block_select_kernel");
}

}  // namespace h3a
