// LUT arithmetic of the block-sparse kernels: which key block a stage of a
// LUT row belongs to and which key it starts at.  Host and device code, so
// that the arithmetic can be checked exhaustively on the CPU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace h3a {

constexpr int kLutStageKeys = 64;  // keys per stage

// Key block of stage t of a LUT row, where a key block is sub = 1..4 stages:
// t / sub, the division by 3 as a multiply-high (exact for 0 <= t < 2^31).
__host__ __device__ __forceinline__ int block_of_stage(int t, int sub) {
  return sub == 3 ? (int)(((uint64_t)(uint32_t)t * 0x55555556u) >> 32) : t >> (sub >> 1);
}

// The same without a branch on sub: t / sub = high 32 bits of (2t) * magic,
// magic = ceil(2^31 / sub) for sub = 1, 2, 4 (exact powers of two) and
// ceil(2^32 / 6) = (2^32 + 2) / 6 = 0x2AAAAAAB for sub = 3, where
// 2t * magic / 2^32 = (t / 3)(1 + 2^-31), whose floor is t / 3 for
// 0 <= t < 2^31.  stage_magic is computed once per work
// item; block_of_stage_magic is one shift and one multiply-high.
__host__ __device__ __forceinline__ uint32_t stage_magic(int sub) {
  return sub == 3 ? 0x2AAAAAABu : 0x80000000u >> (sub >> 1);
}
__host__ __device__ __forceinline__ int block_of_stage_magic(int t, uint32_t magic) {
  return (int)(((uint64_t)((uint32_t)t << 1) * magic) >> 32);
}

// First key of stage t of a LUT row whose entry for that stage's block is
// kb, or Skv (a stage that loads nothing and is fully masked) when kb names
// no key block (kb < 0 or kb >= nkb = ceil(Skv / blk_k)).  kb is checked
// before any multiply, so kb * blk_k < Skv and nothing overflows for any
// 32-bit kb and Skv <= INT_MAX - 256.
__host__ __device__ __forceinline__ int lut_stage_key0(int t, int kb, int nkb, int blk_k, int sub, int Skv) {
  if ((uint32_t)kb >= (uint32_t)nkb) return Skv;
  const int key0 = kb * blk_k + (t - block_of_stage(t, sub) * sub) * kLutStageKeys;
  return key0 < Skv ? key0 : Skv;
}
// The same with the block from block_of_stage_magic (magic = stage_magic(sub))
// and the range checks as selects; the key is formed in unsigned arithmetic
// (it only wraps for a kb that is then discarded).
__host__ __device__ __forceinline__ int lut_stage_key0_sel(int t, int kb, int nkb, int blk_k, int sub,
                                                           uint32_t magic, int Skv) {
  const uint32_t off = (uint32_t)(t - block_of_stage_magic(t, magic) * sub) * (uint32_t)kLutStageKeys;
  const int key0 = (int)((uint32_t)kb * (uint32_t)blk_k + off);
  return (uint32_t)kb >= (uint32_t)nkb ? Skv : (key0 < Skv ? key0 : Skv);
}

// The same as pure arithmetic, with the block from block_of_stage_magic
// (magic = stage_magic(sub)): an entry outside [0, nkb) is replaced by nkb,
// whose first key nkb * blk_k is already >= Skv, so the final min with Skv
// gives Skv for it.  Unsigned, so nothing overflows for Skv <= INT_MAX - 256
// (nkb * blk_k + off < Skv + 2 * blk_k < 2^32).
__host__ __device__ __forceinline__ int lut_stage_key0_magic(int t, int kb, int nkb, int blk_k, int sub,
                                                             uint32_t magic, int Skv) {
  const uint32_t off = (uint32_t)(t - block_of_stage_magic(t, magic) * sub) * (uint32_t)kLutStageKeys;
  const uint32_t kbc = (uint32_t)kb < (uint32_t)nkb ? (uint32_t)kb : (uint32_t)nkb;
  const uint32_t key0 = kbc * (uint32_t)blk_k + off;
  return (int)(key0 < (uint32_t)Skv ? key0 : (uint32_t)Skv);
}

}  // namespace h3a
