// Block-map construction for the block-sparse (h3_sla) path, on the GPU.
//
// The reference gets its block map from SLA's get_block_map
// (custom_nodes/h3_sla/__init__.py:232): mean-pool q and k over blocks of
// rows, score every (query block, key block) pair by the dot product of the
// pooled vectors, keep the top-k key blocks of each query block.  Here:
//   block_pool_kernel   : bf16 [B,H,S,128] (strided) -> fp32 block means
//                         [B,H,ceil(S/blk),128], over the valid rows of each
//                         block.  HBM-bound: reads the tensor once.
//   block_select_kernel : one workgroup per (b,h,query block): scores against
//                         all key blocks into LDS, rank by (score desc, index
//                         asc), keep rank < keep plus the optional diagonal,
//                         and write the kept indices in ascending order (the
//                         LUT h3a_attn_fwd_blocksparse consumes), the count,
//                         and optionally the 0/1 map.
// Centring k by its sequence mean (SLA's K smoothing) shifts every score of a
// row by the same amount, so it never changes the selection and is not needed.
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

__global__ void __launch_bounds__(kSelThreads) block_select_kernel(
    const float *pq, const float *pk, int nq, int nk, int keep, int force_diag, int blk_q,
    int blk_k, int32_t *lut, int32_t *counts, int max_k, uint8_t *map) {
  extern __shared__ float sel_lds[];
  float *sc = sel_lds;                       // [nk] scores
  float *q = sel_lds + nk;                   // [128] pooled query block
  int *flag = (int *)(sel_lds + nk + kPoolD);  // [nk] kept flags
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;            // (b*H + h)*nq + i
  const int i = (int)(row % nq);
  const int64_t bh = row / nq;
  const float *pkh = pk + bh * (int64_t)nk * kPoolD;
  if (tid < kPoolD) q[tid] = pq[row * kPoolD + tid];
  __syncthreads();
  for (int j = tid; j < nk; j += kSelThreads) {
    const float *kr = pkh + (int64_t)j * kPoolD;
    float acc = 0.f;
#pragma unroll 8
    for (int d = 0; d < kPoolD; d += 4) {
      const float4 kv = *(const float4 *)(kr + d);
      acc = fmaf(q[d], kv.x, acc);
      acc = fmaf(q[d + 1], kv.y, acc);
      acc = fmaf(q[d + 2], kv.z, acc);
      acc = fmaf(q[d + 3], kv.w, acc);
    }
    sc[j] = acc;
  }
  __syncthreads();
  const int diag = (int)(((int64_t)i * blk_q) / blk_k);
  for (int j = tid; j < nk; j += kSelThreads) {
    const float v = sc[j];
    int rank = 0;
    for (int t = 0; t < nk; ++t) {
      const float u = sc[t];
      rank += (u > v) || (u == v && t < j);
    }
    flag[j] = (rank < keep) || (force_diag && j == diag);
  }
  __syncthreads();
  int32_t *out = lut + row * max_k;
  for (int j = tid; j < nk; j += kSelThreads) {
    if (map) map[row * nk + j] = (uint8_t)flag[j];
    if (flag[j]) {
      int pos = 0;
      for (int t = 0; t < j; ++t) pos += flag[t];
      if (pos < max_k) out[pos] = j;
    }
  }
  if (tid == 0) {
    int total = 0;
    for (int t = 0; t < nk; ++t) total += flag[t];
    const int kept = total < max_k ? total : max_k;
    counts[row] = kept;
    for (int t = kept; t < max_k; ++t) out[t] = -1;
  }
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
  const size_t lds = (size_t)(2 * nk + kPoolD) * sizeof(float);
  hipLaunchKernelGGL(block_select_kernel, dim3((unsigned)((int64_t)B * H * nq)), dim3(kSelThreads), lds,
                     s, pq, pk, nq, nk, keep, force_diag, blk_q, blk_k, lut, counts, max_k, map);
  return check_launch("block_select_kernel");
}

}  // namespace h3a
