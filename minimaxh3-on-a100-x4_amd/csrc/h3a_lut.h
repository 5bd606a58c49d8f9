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

}  // namespace h3a
