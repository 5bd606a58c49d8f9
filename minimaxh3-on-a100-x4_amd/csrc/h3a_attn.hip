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
//  * Workgroup = NW waves x 32 query rows (BM = 32*NW).  Each wave keeps its
//    32 query rows as the B operand of v_mfma_f32_32x32x16_bf16 in VGPRs.
//  * The score tile is produced transposed, S^T = K Q^T, so every lane owns a
//    single query row (column l%32) and 32 of the 64 keys of a stage.  Row
//    max is an in-register reduction plus one v_permlane32_swap with the
//    partner lane; the row sum needs no cross-lane traffic until the end.
//  * That layout is already the B operand of O^T += V^T P^T: the P tile goes
//    from the score accumulators straight into the PV MFMA (no LDS round
//    trip).  V is staged transposed in LDS with keys ordered to match the
//    score accumulator's key order (see vt_pos).
//  * K/V stages of 64 keys are double-buffered in LDS; the next stage is
//    fetched with 128-bit global loads into registers while the current one
//    is consumed, so one barrier per stage suffices.
//  * exp2-based softmax with scale*log2(e) folded into one FMA.
//  * Workgroup ids are remapped XCD-aware (xcd_remap).
#include "h3a_device.h"
#include "h3a_internal.h"

namespace h3a {

constexpr int kD = 128;
constexpr int kBN = 64;             // keys per pipeline stage
constexpr int kKStride = kD + 8;    // K stage row stride in LDS (elements), padded
constexpr int kVtStride = kBN;      // V^T stage row stride (elements), chunk-swizzled

// ---------------------------------------------------------------------------
// V^T stage layout.  For the PV product the k-slot (g = lane/32, e = 0..7)
// of 16-key step ks carries key 16*ks + 8*(e/4) + 4*g + e%4 (the order in
// which the S^T accumulator holds keys).  Storing key k of a stage at
// position vt_pos(k) (bits 2 and 3 swapped) makes the 8 keys one lane needs
// contiguous: positions 16*ks + 8*g .. +7.
__device__ __forceinline__ int vt_pos(int key) {
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}
// 16-byte chunk swizzle of a V^T row: conflict-free 128-bit reads by 8
// consecutive rows and 64-bit transposing writes by rows 8 apart.
__device__ __forceinline__ int vt_swz(int d) { return (d + (d >> 3)) & 7; }
__device__ __forceinline__ int vt_off(int d, int pos) {
  return d * kVtStride + ((((pos >> 3) ^ vt_swz(d)) << 3) | (pos & 7));
}

// One 64-key K/V stage moving HBM -> registers -> LDS.
template <int NT>
struct KvStage {
  static constexpr int KL = (kBN * kD / 8) / NT;         // 16-byte K chunks per thread
  static constexpr int VL = (kBN / 4) * (kD / 8) / NT;   // (4-key, 8-dim) V blocks per thread
  static_assert(KL * NT == kBN * kD / 8, "K stage must split evenly");
  static_assert(VL * NT == (kBN / 4) * (kD / 8), "V stage must split evenly");
  u32x4 kr[KL];
  u32x4 vr[VL][4];

  // Rows >= Skv (or < 0) load as zeros so masked keys never carry NaN/Inf.
  __device__ __forceinline__ void load(const uint16_t *Kb, int64_t kss, const uint16_t *Vb,
                                       int64_t vss, int key0, int Skv, int tid) {
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const int idx = tid + i * NT, row = idx >> 4, ch = idx & 15, key = key0 + row;
      kr[i] = (key >= 0 && key < Skv) ? *(const u32x4 *)(Kb + (int64_t)key * kss + ch * 8)
                                      : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int idx = tid + i * NT, kq = idx >> 4, dc = idx & 15;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = key0 + 4 * kq + r;
        vr[i][r] = (key >= 0 && key < Skv) ? *(const u32x4 *)(Vb + (int64_t)key * vss + dc * 8)
                                           : u32x4{0, 0, 0, 0};
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t *sK, uint16_t *sVt, int tid) const {
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const int idx = tid + i * NT, row = idx >> 4, ch = idx & 15;
      *(u32x4 *)(sK + row * kKStride + ch * 8) = kr[i];
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int idx = tid + i * NT, kq = idx >> 4, dc = idx & 15;
      const int pos0 = vt_pos(4 * kq);  // 4 consecutive keys stay consecutive
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int w = j >> 1;
        const uint32_t a0 = vr[i][0][w], a1 = vr[i][1][w], a2 = vr[i][2][w], a3 = vr[i][3][w];
        u32x2 val;
        if (j & 1) {
          val.x = (a0 >> 16) | (a1 & 0xffff0000u);
          val.y = (a2 >> 16) | (a3 & 0xffff0000u);
        } else {
          val.x = (a0 & 0xffffu) | (a1 << 16);
          val.y = (a2 & 0xffffu) | (a3 << 16);
        }
        *(u32x2 *)(sVt + vt_off(dc * 8 + j, pos0)) = val;
      }
    }
  }
};

// S^T (64 keys x 32 queries of this wave) = K_stage Q^T.  s0: keys 0-31, s1: 32-63.
__device__ __forceinline__ void score_tile(const uint16_t *kbuf, const u32x4 (&qf)[8], int l32,
                                           int g, f32x16 &s0, f32x16 &s1) {
  s0 = f32x16{0.f};
  s1 = f32x16{0.f};
  const uint16_t *r0 = kbuf + l32 * kKStride + 8 * g;
  const uint16_t *r1 = r0 + 32 * kKStride;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const u32x4 a0 = *(const u32x4 *)(r0 + ks * 16);
    const u32x4 a1 = *(const u32x4 *)(r1 + ks * 16);
    s0 = mfma_32x32x16(a0, qf[ks], s0);
    s1 = mfma_32x32x16(a1, qf[ks], s1);
  }
}

// P^T fragments for the 4 sixteen-key steps, straight from the S^T registers.
__device__ __forceinline__ void pack_p(const f32x16 &s0, const f32x16 &s1, u32x4 (&pf)[4]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    pf[h] = u32x4{pack_bf16x2(s0[8 * h + 0], s0[8 * h + 1]), pack_bf16x2(s0[8 * h + 2], s0[8 * h + 3]),
                  pack_bf16x2(s0[8 * h + 4], s0[8 * h + 5]), pack_bf16x2(s0[8 * h + 6], s0[8 * h + 7])};
    pf[2 + h] = u32x4{pack_bf16x2(s1[8 * h + 0], s1[8 * h + 1]), pack_bf16x2(s1[8 * h + 2], s1[8 * h + 3]),
                      pack_bf16x2(s1[8 * h + 4], s1[8 * h + 5]), pack_bf16x2(s1[8 * h + 6], s1[8 * h + 7])};
  }
}

// O^T (128 dims x 32 queries) += V^T_stage P^T.
__device__ __forceinline__ void pv_tile(const uint16_t *vbuf, const u32x4 (&pf)[4], int l32, int g,
                                        f32x16 (&o)[4]) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const u32x4 av = *(const u32x4 *)(vbuf + vt_off(dt * 32 + l32, ks * 16 + 8 * g));
      o[dt] = mfma_32x32x16(av, pf[ks], o[dt]);
    }
  }
}

template <int NW, bool kSparse>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
attn_fwd_kernel(AttnArgs a) {
  constexpr int NT = NW * 64;
  constexpr int BM = NW * 32;
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][kBN * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[2][kD * kVtStride];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;

  const int w = xcd_remap(blockIdx.x, a.total);
  const int qt = w % a.nqt, bh = w / a.nqt;
  const int h = bh % a.H, b = bh / a.H;

  const uint16_t *Qb = a.q + b * a.qsb + h * a.qsh;
  const uint16_t *Kb = a.k + b * a.ksb + h * a.ksh;
  const uint16_t *Vb = a.v + b * a.vsb + h * a.vsh;
  uint16_t *Ob = a.o + b * a.osb + h * a.osh;

  int niter;
  const int32_t *lut_row = nullptr;
  if constexpr (kSparse) {
    const int64_t row = (int64_t)bh * a.nqt + qt;
    const int cnt = a.counts[row];
    niter = (cnt < 0 ? 0 : (cnt > a.lut_stride ? a.lut_stride : cnt)) * a.sub;
    lut_row = a.lut + row * a.lut_stride;
  } else {
    niter = (a.Skv + kBN - 1) / kBN;
  }
  // First key of stage j.  A LUT entry outside the key range maps to Skv:
  // the stage then loads nothing and is fully masked.
  auto key_base = [&](int j) -> int {
    if constexpr (kSparse) {
      const int kb = lut_row[j / a.sub];
      const int key0 = kb * a.blk_k + (j % a.sub) * kBN;
      return (kb < 0 || key0 >= a.Skv) ? a.Skv : key0;
    } else {
      return j * kBN;
    }
  };

  const int qrow = qt * BM + wave * 32 + l32;
  u32x4 qf[8];
  if (qrow < a.Sq) {
    const uint16_t *p = Qb + (int64_t)qrow * a.qss + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = *(const u32x4 *)(p + ks * 16);
  } else {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = u32x4{0, 0, 0, 0};
  }

  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{0.f};
  float m = kNegInf;  // running row max, in scale*log2(e) units
  float lsum = 0.f;   // this lane's share of the running row sum

  KvStage<NT> st;
  if (niter > 0) {
    st.load(Kb, a.kss, Vb, a.vss, key_base(0), a.Skv, tid);
    st.store(sK[0], sVt[0], tid);
  }
  __syncthreads();

  for (int j = 0; j < niter; ++j) {
    const int buf = j & 1;
    const int key0 = key_base(j);
    if (j + 1 < niter) st.load(Kb, a.kss, Vb, a.vss, key_base(j + 1), a.Skv, tid);

    f32x16 s0, s1;
    score_tile(sK[buf], qf, l32, g, s0, s1);

    if (key0 + kBN > a.Skv) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = key0 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (kk >= a.Skv) s0[r] = kNegInf;
        if (kk + 32 >= a.Skv) s1[r] = kNegInf;
      }
    }

    float mx = fmaxf(s0[0], s1[0]);
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
    mx = half_swap_max(mx);
    const float mnew = fmaxf(m, mx * a.sl2);
    const float muse = (mnew == kNegInf) ? 0.f : mnew;
    const float alpha = fast_exp2(m - muse);
    m = mnew;

    float rs = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s0[r] = fast_exp2(fmaf(s0[r], a.sl2, -muse));
      s1[r] = fast_exp2(fmaf(s1[r], a.sl2, -muse));
      rs += s0[r] + s1[r];
    }
    lsum = fmaf(lsum, alpha, rs);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;

    u32x4 pf[4];
    pack_p(s0, s1, pf);
    pv_tile(sVt[buf], pf, l32, g, o);

    if (j + 1 < niter) st.store(sK[buf ^ 1], sVt[buf ^ 1], tid);
    __syncthreads();
  }

  const float ltot = half_swap_sum(lsum);
  const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
  if (qrow < a.Sq) {
    uint16_t *p = Ob + (int64_t)qrow * a.oss + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const u32x2 val = {pack_bf16x2(o[dt][4 * rr + 0] * inv, o[dt][4 * rr + 1] * inv),
                           pack_bf16x2(o[dt][4 * rr + 2] * inv, o[dt][4 * rr + 3] * inv)};
        *(u32x2 *)(p + dt * 32 + 8 * rr) = val;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Fragment tests: one wave, the same staging and fragment code as above.
__global__ void __launch_bounds__(64) test_qk_kernel(const uint16_t *Q, const uint16_t *K, float *S) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[kBN * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[kD * kVtStride];
  const int tid = threadIdx.x, g = tid >> 5, l32 = tid & 31;
  KvStage<64> st;
  st.load(K, kD, K, kD, 0, kBN, tid);
  st.store(sK, sVt, tid);
  __syncthreads();
  u32x4 qf[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) qf[ks] = *(const u32x4 *)(Q + l32 * kD + ks * 16 + 8 * g);
  f32x16 s0, s1;
  score_tile(sK, qf, l32, g, s0, s1);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int key = 8 * (r >> 2) + 4 * g + (r & 3);
    S[l32 * kBN + key] = s0[r];
    S[l32 * kBN + key + 32] = s1[r];
  }
}

__global__ void __launch_bounds__(64) test_pv_kernel(const uint16_t *P, const uint16_t *V, float *O) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[kBN * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[kD * kVtStride];
  const int tid = threadIdx.x, g = tid >> 5, l32 = tid & 31;
  KvStage<64> st;
  st.load(V, kD, V, kD, 0, kBN, tid);
  st.store(sK, sVt, tid);
  __syncthreads();
  // Place P[q][key] where the score accumulators would hold it.
  f32x16 s0, s1;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int key = 8 * (r >> 2) + 4 * g + (r & 3);
    s0[r] = __uint_as_float((uint32_t)P[l32 * kBN + key] << 16);
    s1[r] = __uint_as_float((uint32_t)P[l32 * kBN + key + 32] << 16);
  }
  u32x4 pf[4];
  pack_p(s0, s1, pf);
  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{0.f};
  pv_tile(sVt, pf, l32, g, o);
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
int launch_attn_dense(const AttnArgs &a, hipStream_t s) {
  hipLaunchKernelGGL((attn_fwd_kernel<4, false>), dim3(a.total), dim3(256), 0, s, a);
  return check_launch("attn_fwd_kernel<dense>");
}

int launch_attn_sparse(const AttnArgs &a, int blk_q, hipStream_t s) {
  if (blk_q == 128) {
    hipLaunchKernelGGL((attn_fwd_kernel<4, true>), dim3(a.total), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((attn_fwd_kernel<2, true>), dim3(a.total), dim3(128), 0, s, a);
  }
  return check_launch("attn_fwd_kernel<sparse>");
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

int attn_kernel_attrs(int which, double out[6]) {
  switch (which) {
    case H3A_KERNEL_ATTN_DENSE:
      return fill_attrs(reinterpret_cast<const void *>(&attn_fwd_kernel<4, false>), 256, out);
    case H3A_KERNEL_ATTN_SPARSE_128:
      return fill_attrs(reinterpret_cast<const void *>(&attn_fwd_kernel<4, true>), 256, out);
    case H3A_KERNEL_ATTN_SPARSE_64:
      return fill_attrs(reinterpret_cast<const void *>(&attn_fwd_kernel<2, true>), 128, out);
    default:
      return fail(H3A_ERR_INVALID_ARG, "unknown kernel id %d", which);
  }
}

}  // namespace h3a
