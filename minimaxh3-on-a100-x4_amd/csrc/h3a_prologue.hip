// Fused per-head qk-RMSNorm + split-half RoPE, in place, for gfx950.
//
// Replaces comfy_kitchen's rms_rope_split_half_(q, k, rope_freqs, qw, kw,
// epsilon, rot_dim) as called by the DiT attention (harness/sp_runtime.py:93-99,
// custom_nodes/h3_profiler/__init__.py:99-106) on [1,S,H,128] strided views of
// the fused QKV projection output.  It is HBM-bound: every q/k row is read
// once and written once (4*S*H*D*2 bytes) plus one rope row per token.
//
// Layout of the work: one wave owns one (b,s) token and a chunk of HPW heads
// (28 or 16, chosen per launch).  Its four 16-lane groups walk the chunk
// one head each per step; within a group each lane holds 8 consecutive dims
// (one 128-bit access), so one wave access moves four whole 256-byte head rows
// (1 KB contiguous in the fused QKV layout).  The token's RoPE matrices and
// the two weight vectors are loaded into registers once per wave and reused
// for all 2 x HPW rows; the chunk's row loads are issued before any math.  The sum of squares
// is reduced across the 16 lanes with xor shuffles; the RoPE partner dims
// (i, i+rot/2) sit rot/16 lanes apart and are fetched with one shuffle each.
#include "h3a_device.h"
#include "h3a_internal.h"

namespace h3a {

constexpr int kRopeD = 128;

__device__ __forceinline__ float group16_sum(float v) {
  v += __shfl_xor(v, 1, 16);
  v += __shfl_xor(v, 2, 16);
  v += __shfl_xor(v, 4, 16);
  v += __shfl_xor(v, 8, 16);
  return v;
}

__device__ __forceinline__ void unpack8(const u32x4 &w, float (&x)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = bf16_lo(w[i]);
    x[2 * i + 1] = bf16_hi(w[i]);
  }
}

__device__ __forceinline__ u32x4 pack8(const float (&x)[8]) {
  return u32x4{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(x[4], x[5]),
               pack_bf16x2(x[6], x[7])};
}

// Heads per wave (HPW, a multiple of 4: four 16-lane groups): 28 when it
// divides H, otherwise 16.  At H=56, 28 gives two full waves per token, each
// reading the token's RoPE row once (same box: 5.41 TB/s against 5.15 with 16
// heads, of which the fourth wave per token has 8; 4.80 with 8 full waves and
// 5.00 with one wave of all 56, whose 201 VGPRs halve the waves in flight);
// non-temporal stores changed nothing.
__host__ __device__ constexpr int rope_heads_per_wave(int H) { return H % 28 == 0 ? 28 : 16; }

// y = rmsnorm(x) * w, then rotate pairs (i, i+rot/2) with the lane's 2x2 matrices.
__device__ __forceinline__ void norm_rope_row(float (&x)[8], const float (&w)[8], float eps,
                                              const float4 (&R)[8], int c, int rot) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
  ss = group16_sum(ss);
  const float r = rsqrtf(ss * (1.0f / kRopeD) + eps);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = x[e] * r * w[e];

  const int nh = rot >> 4;  // lanes holding the first half of the rotated dims
  const bool first = c < nh;
  const bool rotated = c < 2 * nh;
  const int partner = first ? c + nh : (rotated ? c - nh : c);
  float xp[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) xp[e] = __shfl(x[e], partner, 16);
  if (rotated) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      x[e] = first ? fmaf(R[e].x, x[e], R[e].y * xp[e]) : fmaf(R[e].z, xp[e], R[e].w * x[e]);
  }
}

template <int kHeadsPerWave>
__global__ void __launch_bounds__(256) qk_rmsnorm_rope_kernel(RopeArgs a) {
  static_assert(kHeadsPerWave % 4 == 0, "four 16-lane groups per wave");
  constexpr int kSteps = kHeadsPerWave / 4;  // heads per 16-lane group
  const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4, c = lane & 15;
  const int nchunk = (a.H + kHeadsPerWave - 1) / kHeadsPerWave;
  const int64_t item = (int64_t)blockIdx.x * 4 + (tid >> 6);  // (token, head chunk)
  if (item >= (int64_t)a.B * a.S * nchunk) return;            // whole waves leave together
  const int chunk = (int)(item % nchunk);
  const int64_t bs = item / nchunk;
  const int s = (int)(bs % a.S), b = (int)(bs / a.S);

  float wq[8], wk[8];
  unpack8(*(const u32x4 *)(a.qw + c * 8), wq);
  unpack8(*(const u32x4 *)(a.kw + c * 8), wk);
  float4 R[8];
  const int nh = a.rot >> 4;
  if (c < 2 * nh) {
    const float *rope_row = a.rope + b * a.rsb + s * a.rss + (c < nh ? c : c - nh) * 8 * 4;
#pragma unroll
    for (int e = 0; e < 8; ++e) R[e] = *(const float4 *)(rope_row + e * 4);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) R[e] = float4{1.f, 0.f, 0.f, 1.f};
  }

  uint16_t *qrow = a.q + b * a.qsb + s * a.qss + c * 8;
  uint16_t *krow = a.k + b * a.ksb + s * a.kss + c * 8;
  int heads[kSteps];
  u32x4 qv[kSteps], kv[kSteps];
#pragma unroll
  for (int i = 0; i < kSteps; ++i) {
    const int h = chunk * kHeadsPerWave + i * 4 + grp;
    heads[i] = h;
    const int hc = h < a.H ? h : a.H - 1;  // past-the-end groups recompute the last head, store nothing
    qv[i] = *(const u32x4 *)(qrow + hc * a.qsh);
    kv[i] = *(const u32x4 *)(krow + hc * a.ksh);
  }
#pragma unroll
  for (int i = 0; i < kSteps; ++i) {
    float xq[8], xk[8];
    unpack8(qv[i], xq);
    unpack8(kv[i], xk);
    norm_rope_row(xq, wq, a.eps, R, c, a.rot);
    norm_rope_row(xk, wk, a.eps, R, c, a.rot);
    if (heads[i] < a.H) {
      *(u32x4 *)(qrow + heads[i] * a.qsh) = pack8(xq);
      *(u32x4 *)(krow + heads[i] * a.ksh) = pack8(xk);
    }
  }
}

// The prologue with the block pooling of SLA's block map fused in (the
// means block_pool_kernel takes of the stored q and k).  One workgroup per
// (b, block of blk tokens, chunk of kHeadsPerWave heads); wave w normalises
// and rotates tokens w, w+4, w+8, ... of the block as qk_rmsnorm_rope_kernel
// does and sums, per (head, dim), the bf16 values it stores, in token order.
// The waves' sums S0..S3 are combined as (S0 + S1) + (S2 + S3) through LDS and
// scaled by 1/rows: block_pool_kernel's lane rg sums rows rg, rg+4, ... in
// order and combines the four lane groups in that association, so the means
// are equal to its output bit for bit, and the selection made from them is
// the same.
template <int kHeadsPerWave>
__global__ void __launch_bounds__(256) qk_rmsnorm_rope_pool_kernel(RopeArgs a, int blk, int nb, float *pq,
                                                                   float *pk) {
  static_assert(kHeadsPerWave % 4 == 0, "four 16-lane groups per wave");
  constexpr int kSteps = kHeadsPerWave / 4;
  // Partial sums of waves 1 and 3 (slots 0 and 1), then of wave 2 (slot 0):
  // [slot][step][q,k][lane] of 8 floats.
  __shared__ __attribute__((aligned(16))) float xch[2][kSteps][2][64][8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, grp = lane >> 4, c = lane & 15;
  const int nchunk = (a.H + kHeadsPerWave - 1) / kHeadsPerWave;
  const int chunk = (int)(blockIdx.x % nchunk);
  const int64_t bj = blockIdx.x / nchunk;
  const int j = (int)(bj % nb), b = (int)(bj / nb);
  const int r0 = j * blk;
  const int rows = a.S - r0 < blk ? a.S - r0 : blk;

  float wq[8], wk[8];
  unpack8(*(const u32x4 *)(a.qw + c * 8), wq);
  unpack8(*(const u32x4 *)(a.kw + c * 8), wk);
  const int nh = a.rot >> 4;
  int heads[kSteps];
#pragma unroll
  for (int i = 0; i < kSteps; ++i) heads[i] = chunk * kHeadsPerWave + i * 4 + grp;
  float sq[kSteps][8], sk[kSteps][8];
#pragma unroll
  for (int i = 0; i < kSteps; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) sq[i][e] = sk[i][e] = 0.f;

  for (int t = wave; t < rows; t += 4) {
    const int s = r0 + t;
    float4 R[8];
    if (c < 2 * nh) {
      const float *rope_row = a.rope + b * a.rsb + s * a.rss + (c < nh ? c : c - nh) * 8 * 4;
#pragma unroll
      for (int e = 0; e < 8; ++e) R[e] = *(const float4 *)(rope_row + e * 4);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) R[e] = float4{1.f, 0.f, 0.f, 1.f};
    }
    uint16_t *qrow = a.q + b * a.qsb + s * a.qss + c * 8;
    uint16_t *krow = a.k + b * a.ksb + s * a.kss + c * 8;
    u32x4 qv[kSteps], kv[kSteps];
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      const int hc = heads[i] < a.H ? heads[i] : a.H - 1;  // past-the-end groups store nothing
      qv[i] = *(const u32x4 *)(qrow + hc * a.qsh);
      kv[i] = *(const u32x4 *)(krow + hc * a.ksh);
    }
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      float xq[8], xk[8];
      unpack8(qv[i], xq);
      unpack8(kv[i], xk);
      norm_rope_row(xq, wq, a.eps, R, c, a.rot);
      norm_rope_row(xk, wk, a.eps, R, c, a.rot);
      const u32x4 oq = pack8(xq), ok = pack8(xk);
      if (heads[i] < a.H) {
        *(u32x4 *)(qrow + heads[i] * a.qsh) = oq;
        *(u32x4 *)(krow + heads[i] * a.ksh) = ok;
      }
      float yq[8], yk[8];  // the stored values
      unpack8(oq, yq);
      unpack8(ok, yk);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sq[i][e] += yq[e];
        sk[i][e] += yk[e];
      }
    }
  }

  auto put = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
      *(float4 *)&xch[slot][i][0][lane][0] = float4{sq[i][0], sq[i][1], sq[i][2], sq[i][3]};
      *(float4 *)&xch[slot][i][0][lane][4] = float4{sq[i][4], sq[i][5], sq[i][6], sq[i][7]};
      *(float4 *)&xch[slot][i][1][lane][0] = float4{sk[i][0], sk[i][1], sk[i][2], sk[i][3]};
      *(float4 *)&xch[slot][i][1][lane][4] = float4{sk[i][4], sk[i][5], sk[i][6], sk[i][7]};
    }
  };
  auto add = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kSteps; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sq[i][e] += xch[slot][i][0][lane][e];
        sk[i][e] += xch[slot][i][1][lane][e];
      }
  };
  if (wave & 1) put(wave >> 1);  // S1 -> slot 0, S3 -> slot 1
  __syncthreads();
  if (!(wave & 1)) add(wave >> 1);  // wave 0: S0 + S1, wave 2: S2 + S3
  __syncthreads();
  if (wave == 2) put(0);
  __syncthreads();
  if (wave != 0) return;  // no barrier follows
  add(0);  // (S0 + S1) + (S2 + S3)
  const float inv = 1.f / (float)rows;
#pragma unroll
  for (int i = 0; i < kSteps; ++i) {
    if (heads[i] >= a.H) continue;
    const int64_t o = (((int64_t)b * a.H + heads[i]) * nb + j) * kRopeD + c * 8;
    *(float4 *)(pq + o) = float4{sq[i][0] * inv, sq[i][1] * inv, sq[i][2] * inv, sq[i][3] * inv};
    *(float4 *)(pq + o + 4) = float4{sq[i][4] * inv, sq[i][5] * inv, sq[i][6] * inv, sq[i][7] * inv};
    *(float4 *)(pk + o) = float4{sk[i][0] * inv, sk[i][1] * inv, sk[i][2] * inv, sk[i][3] * inv};
    *(float4 *)(pk + o + 4) = float4{sk[i][4] * inv, sk[i][5] * inv, sk[i][6] * inv, sk[i][7] * inv};
  }
}

int launch_qk_rmsnorm_rope_pool(const RopeArgs &a, int blk, float *pq, float *pk, hipStream_t s) {
  constexpr int kHpw = 8;
  const int nb = (a.S + blk - 1) / blk;
  const int64_t wgs = (int64_t)a.B * nb * ((a.H + kHpw - 1) / kHpw);
  hipLaunchKernelGGL(qk_rmsnorm_rope_pool_kernel<kHpw>, dim3((unsigned)wgs), dim3(256), 0, s, a, blk, nb, pq, pk);
  return check_launch("qk_rmsnorm_rope_pool_kernel");
}

int launch_qk_rmsnorm_rope(const RopeArgs &a, hipStream_t s) {
  const int hpw = rope_heads_per_wave(a.H);
  const int64_t items = (int64_t)a.B * a.S * ((a.H + hpw - 1) / hpw);
  const int64_t blocks = (items + 3) / 4;
  if (hpw == 28)
    hipLaunchKernelGGL(qk_rmsnorm_rope_kernel<28>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(qk_rmsnorm_rope_kernel<16>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_launch("qk_rmsnorm_rope_kernel");
}

int rope_kernel_attrs(double out[6]) {
  hipFuncAttributes fa;
  const void *fn = reinterpret_cast<const void *>(&qk_rmsnorm_rope_kernel<28>);  // the H=56 width
  if (hipFuncGetAttributes(&fa, fn) != hipSuccess) return fail(H3A_ERR_HIP, "hipFuncGetAttributes failed");
  int blocks = 0, dev = 0, clk = 0, max_threads = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, 256, 0) != hipSuccess ||
      hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&clk, hipDeviceAttributeClockRate, dev) != hipSuccess ||
      hipDeviceGetAttribute(&max_threads, hipDeviceAttributeMaxThreadsPerMultiProcessor, dev) != hipSuccess)
    return fail(H3A_ERR_HIP, "occupancy query failed");
  out[0] = fa.numRegs;
  out[1] = (double)fa.sharedSizeBytes;
  out[2] = blocks;
  out[3] = clk;
  out[4] = max_threads > 0 ? (double)(blocks * 256) / max_threads : 0.0;
  out[5] = 256;
  return H3A_OK;
}

}  // namespace h3a
