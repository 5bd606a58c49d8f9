// Exhaustive/edge-case check of the block-sparse LUT arithmetic
// (minimaxh3-on-a100-x4_amd/csrc/h3a_lut.h) on the host, against int64 math.
// Built and run by tests/test_lut_arith.py; prints "OK" or the first mismatch.
#include <climits>
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#include "h3a_lut.h"

static int key0_ref(int64_t t, int64_t kb, int64_t Skv, int64_t blk_k, int64_t sub) {
  const int64_t nkb = (Skv + blk_k - 1) / blk_k;
  if (kb < 0 || kb >= nkb) return (int)Skv;
  const int64_t key0 = kb * blk_k + (t % sub) * 64;
  return (int)(key0 < Skv ? key0 : Skv);
}

int main() {
  std::mt19937_64 rng(7);
  std::vector<int> ts;
  for (int t = 0; t < 300000; ++t) ts.push_back(t);
  for (int i = 0; i < 2000000; ++i) ts.push_back((int)(rng() & 0x7fffffffu));
  for (int t : {INT_MAX, INT_MAX - 1, INT_MAX - 2, 1 << 30, (1 << 30) + 1, (1 << 30) - 1, 3 << 29})
    ts.push_back(t);
  for (int sub = 1; sub <= 4; ++sub)
    for (int t : ts) {
      if (h3a::block_of_stage(t, sub) != t / sub) {
        printf("block_of_stage(%d, %d) = %d, want %d\n", t, sub, h3a::block_of_stage(t, sub), t / sub);
        return 1;
      }
      if (h3a::block_of_stage_magic(t, h3a::stage_magic(sub)) != t / sub) {
        printf("block_of_stage_magic(%d, %d) = %d, want %d\n", t, sub,
               h3a::block_of_stage_magic(t, h3a::stage_magic(sub)), t / sub);
        return 1;
      }
    }
  const int skvs[] = {1, 63, 64, 65, 127, 129, 255, 257, 42120, 46052, 1 << 24, INT_MAX - 256};
  for (int Skv : skvs)
    for (int blk_k : {64, 128, 192, 256}) {
      const int sub = blk_k / 64;
      const int64_t nkb = ((int64_t)Skv + blk_k - 1) / blk_k;
      std::vector<int64_t> kbs = {-1, -2, INT_MIN, 0, 1, nkb - 1, nkb, nkb + 1, (1 << 24) + 5, INT_MAX,
                                  (int64_t)INT_MAX / blk_k, (int64_t)INT_MAX / blk_k + 1, 1LL << 31 >> 6};
      for (int i = 0; i < 2000; ++i) kbs.push_back((int64_t)(int32_t)(uint32_t)rng());
      for (int i = 0; i < 2000; ++i) kbs.push_back((int64_t)(rng() % (uint64_t)(nkb + 2)) - 1);
      for (int64_t kb64 : kbs) {
        if (kb64 < INT_MIN || kb64 > INT_MAX) continue;
        const int kb = (int)kb64;
        for (int t : {0, 1, 2, 3, 4, 5, 6, 7, 11, 1000, 65535, INT_MAX - 3, INT_MAX}) {
          const int got = h3a::lut_stage_key0(t, kb, (int)nkb, blk_k, sub, Skv);
          const int want = key0_ref(t, kb, Skv, blk_k, sub);
          if (got != want || got < 0 || got > Skv) {
            printf("lut_stage_key0(t=%d, kb=%d, nkb=%lld, blk_k=%d, Skv=%d) = %d, want %d\n", t, kb,
                   (long long)nkb, blk_k, Skv, got, want);
            return 1;
          }
          const int got_m = h3a::lut_stage_key0_magic(t, kb, (int)nkb, blk_k, sub, h3a::stage_magic(sub), Skv);
          const int got_s = h3a::lut_stage_key0_sel(t, kb, (int)nkb, blk_k, sub, h3a::stage_magic(sub), Skv);
          if (got_m != want || got_s != want) {
            printf("lut_stage_key0_magic / _sel(t=%d, kb=%d, nkb=%lld, blk_k=%d, Skv=%d) = %d / %d, want %d\n", t,
                   kb, (long long)nkb, blk_k, Skv, got_m, got_s, want);
            return 1;
          }
        }
      }
    }
  printf("OK\n");
  return 0;
}
