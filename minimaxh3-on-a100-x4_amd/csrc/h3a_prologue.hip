// Fused per-head qk-RMSNorm + split-half RoPE, in place, for gfx950.
//
// Replaces comfy_kitchen's rms_rope_split_half_(q, k, rope_freqs, qw, kw,
// epsilon, rot_dim) as called by the DiT attention (harness/sp_runtime.py:93-99,
// custom_nodes/h3_profiler/__init__.py:99-106) on [1,S,H,128] strided views of
// the fused QKV projection output.  It is HBM-bound: every q/k row is read
// once and written once (4*S*H*D*2 bytes) plus one rope row per token.
//
// Layout of the work: 16 lanes own one (b,s,h) row of q AND the same row of
// k, 8 consecutive dims (one 128-bit access) per lane, so a 64-lane wave moves
// four full 256-byte rows of each tensor per access.  The sum of squares is
// reduced across the 16 lanes with xor shuffles; the RoPE partner dims
// (i, i+rot/2) sit rot/16 lanes apart and are fetched with one shuffle per
// value.
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

// y = rmsnorm(x) * w, then rotate pairs (i, i+rot/2) with the 2x2 matrices.
__device__ __forceinline__ void norm_rope_row(float (&x)[8], const float (&w)[8], float eps,
                                              const float *rope_row, int c, int rot) {
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
    const int i0 = (first ? c : c - nh) * 8;  // frequency index of x[0]
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float4 R = *(const float4 *)(rope_row + (i0 + e) * 4);
      x[e] = first ? fmaf(R.x, x[e], R.y * xp[e]) : fmaf(R.z, xp[e], R.w * x[e]);
    }
  }
}

__global__ void __launch_bounds__(256) qk_rmsnorm_rope_kernel(RopeArgs a) {
  const int tid = threadIdx.x, c = tid & 15;
  const int64_t row = (int64_t)blockIdx.x * 16 + (tid >> 4);
  if (row >= a.rows) return;  // whole 16-lane groups leave together
  const int h = (int)(row % a.H);
  const int64_t bs = row / a.H;
  const int s = (int)(bs % a.S), b = (int)(bs / a.S);

  uint16_t *qp = a.q + b * a.qsb + s * a.qss + h * a.qsh + c * 8;
  uint16_t *kp = a.k + b * a.ksb + s * a.kss + h * a.ksh + c * 8;
  const u32x4 qv = *(const u32x4 *)qp;
  const u32x4 kv = *(const u32x4 *)kp;
  const u32x4 qwv = *(const u32x4 *)(a.qw + c * 8);
  const u32x4 kwv = *(const u32x4 *)(a.kw + c * 8);
  const float *rope_row = a.rot > 0 ? a.rope + b * a.rsb + s * a.rss : nullptr;

  float xq[8], xk[8], wq[8], wk[8];
  unpack8(qv, xq);
  unpack8(kv, xk);
  unpack8(qwv, wq);
  unpack8(kwv, wk);
  norm_rope_row(xq, wq, a.eps, rope_row, c, a.rot);
  norm_rope_row(xk, wk, a.eps, rope_row, c, a.rot);
  *(u32x4 *)qp = pack8(xq);
  *(u32x4 *)kp = pack8(xk);
}

int launch_qk_rmsnorm_rope(const RopeArgs &a, hipStream_t s) {
  const int64_t blocks = (a.rows + 15) / 16;
  hipLaunchKernelGGL(qk_rmsnorm_rope_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_launch("qk_rmsnorm_rope_kernel");
}

int rope_kernel_attrs(double out[6]) {
  hipFuncAttributes fa;
  const void *fn = reinterpret_cast<const void *>(&qk_rmsnorm_rope_kernel);
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
