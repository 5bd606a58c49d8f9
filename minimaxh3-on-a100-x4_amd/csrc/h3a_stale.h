// Bound of the stale-max softmax of the attention kernels: when a stage's p
// sum forces a refresh of the reference max.  Host and device code, so that the
// predicate can be checked on the CPU under the library's compile flags.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace h3a {

// Largest stage p sum (per lane: 32 keys of one query row) accepted without a
// refresh of the stale reference max.  Every p of a stage is then <= 2^16, so
// a row's unnormalised O is bounded by 2 * 2^16 * ceil(Skv/64) * max|v|: it
// stays finite for max|v| < 2^128 / (2^17 * ceil(Skv/64)), about 3.9e30 at
// Skv = 42120 (a max-subtracted softmax with p <= 1 allows up to ~8e33 there).
constexpr float kStaleSumLimit = 0x1p16f;

// True when the stage sum ps (a sum of exp2 values: +0 or more, or NaN) needs
// a refresh: ps > kStaleSumLimit, +inf or NaN.  Compared as bit patterns, which
// order like the values for ps >= +0 and put every NaN above the limit; a
// float compare could be folded to "ps > limit", false for NaN, by a compiler
// allowed to assume no NaNs (the library builds with -fno-honor-nans).  A
// negative ps, which no stage produces, also counts as a refresh.
__host__ __device__ __forceinline__ bool stage_sum_needs_refresh(float ps) {
  return __builtin_bit_cast(uint32_t, ps) > __builtin_bit_cast(uint32_t, kStaleSumLimit);
}

}  // namespace h3a
