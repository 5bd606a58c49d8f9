// Host-side helpers shared by the libh3attn translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "h3attn.h"

namespace h3a {

// Record a formatted message for h3a_last_error() on this thread; returns code.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Map the last HIP launch status to an H3A code (H3A_OK when clean).
int check_launch(const char *what);

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline hipStream_t as_stream(h3a_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Kernel-side argument block of the attention kernels (passed by value).
struct AttnArgs {
  const uint16_t *q, *k, *v;
  uint16_t *o;
  int64_t qsb, qsh, qss;
  int64_t ksb, ksh, kss;
  int64_t vsb, vsh, vss;
  int64_t osb, osh, oss;
  int B, H, Sq, Skv;
  int nqt;    // query tiles per (b,h) (block-sparse: query sub-blocks of 64 or 128 rows)
  int total;  // B*H*nqt workgroups
  float sl2;  // softmax scale * log2(e)
  // block-sparse only
  const int32_t *lut;
  const int32_t *counts;
  int lut_stride;  // max_k_blocks
  int sub;         // 64-key stages per key block (blk_k / 64: 1..4)
  int blk_k;
  int nkb;         // key blocks, ceil(Skv / blk_k): LUT entries outside [0, nkb) name none
  int nqb;         // LUT rows per (b,h), ceil(Sq / blk_q)
  int qmul;        // query sub-blocks per LUT row (blk_q / sub-block height: 1..3)
  // dense split tail (see launch_attn_dense): work items >= split_first are
  // cut into split_pieces key ranges whose partial results go to ws
  int split_first;
  int split_pieces;
  float *ws;
  // dynamic dispatch (persistent grid, per-XCD work queues): the queues'
  // counters, zeroed before the launch; null for one work item per workgroup
  int *sched;
  // tile path: the two 64-row sub-blocks of each pair, [B*H][pairs][2]
  // (tile_pair_map_kernel), or null for sub-blocks 2p and 2p+1
  const int32_t *pair_map;
};

// Block sizes of the block-sparse path: multiples of the 64-key stage up to
// 256.  Query blocks run as sub-blocks of 128 rows (blk_q 128, 256: the pairs
// kernel) or 64 rows (blk_q 64, 192: the key-split kernel); a key block is
// blk_k / 64 stages.
inline bool sparse_block_ok(int blk) { return blk == 64 || blk == 128 || blk == 192 || blk == 256; }
// Block sizes of a block map that h3a_block_map_to_tile_lut converts: any
// positive multiple of 16 (each 16x16 sub-block of a 32-key column then lies
// in exactly one block pair).
inline bool tile_block_ok(int blk) { return blk > 0 && blk % 16 == 0; }
// 32-key columns a tile LUT entry can name (column << 8 | mask stays positive
// and below 2^24): Skv <= kMaxTileColumns * 32.
constexpr int kMaxTileColumns = 65534;
// Query sub-blocks per (b,h) whose pairing by stage count is sorted in one
// workgroup's LDS (tile path; longer sequences pair sub-blocks 2p, 2p+1).
constexpr int kPairSortMax = 16384;
inline int sparse_sub_block_rows(int blk_q) { return blk_q % 128 == 0 ? 128 : 64; }

// Dense split-tail plan for a problem on the current device.
struct SplitPlan {
  int tiles;    // B*H*query tiles
  int first;    // tiles run whole (the rest are split)
  int pieces;   // key ranges per split tile (1: no split)
  size_t bytes; // workspace bytes (split partials, then the queue counters)
  bool dynamic; // persistent grid with per-XCD work queues
  size_t sched_off;  // byte offset of the queue counters in the workspace
  bool pair_map;     // tile path: sub-blocks paired by stage count (map at offset 0)
};

// Launchers implemented in h3a_attn.hip / h3a_prologue.hip.
int launch_attn_dense(AttnArgs a, hipStream_t s);  // sets nqt/total from its tile height
int plan_attn_split(int B, int H, int Sq, int Skv, SplitPlan *plan);
int launch_attn_dense_split(AttnArgs a, const SplitPlan &plan, void *ws, hipStream_t s);
// tiles: a.lut is a tile LUT (column << 8 | sub-block mask per entry) over
// 64-row query sub-blocks and 32-key columns; blk_q is then ignored.
int launch_attn_sparse(const AttnArgs &a, int blk_q, hipStream_t s, bool tiles = false);
// Block-sparse split tail: pairs of 128-row query blocks play the part of
// the dense tiles (no split for other block heights).
int plan_attn_sparse_split(int B, int H, int Sq, int blk_q, int blk_k, int max_k_blocks, SplitPlan *plan);
int plan_attn_sparse_tiles(int B, int H, int Sq, int max_tiles, SplitPlan *plan);
int launch_attn_sparse_split(const AttnArgs &a, int blk_q, const SplitPlan &plan, void *ws, hipStream_t s,
                             bool tiles = false);
int launch_block_map_to_lut(const uint8_t *map, int B, int H, int nq, int nk, int32_t *lut,
                            int32_t *counts, int max_k_blocks, hipStream_t s);
int launch_block_map_to_tile_lut(const uint8_t *map, int B, int H, int Sq, int Skv, int blk_q, int blk_k,
                                 int32_t *lut, int32_t *counts, int max_tiles, hipStream_t s);
int launch_lut_to_block_map(const int32_t *lut, const int32_t *counts, int B, int H, int nq, int nk,
                            int max_k_blocks, uint8_t *map, hipStream_t s);
int launch_block_pool(const uint16_t *x, const int64_t st[3], int B, int H, int S, int blk,
                      float *out, hipStream_t s);
int launch_block_select(const float *pq, const float *pk, int B, int H, int nq, int nk, int keep,
                        int force_diag, int blk_q, int blk_k, int32_t *lut, int32_t *counts,
                        int max_k, uint8_t *map, hipStream_t s);
int launch_test_qk(const uint16_t *Q, const uint16_t *K, float *S, hipStream_t s);
int launch_test_pv(const uint16_t *P, const uint16_t *V, float *O, hipStream_t s);
int attn_kernel_attrs(int which, double out[6]);
int attn_prof_read(uint64_t *out);  // H3A_PROF_WAVES x H3A_PROF_SLOTS
int attn_prof_reset();

struct RopeArgs {
  uint16_t *q, *k;
  int64_t qsb, qss, qsh;
  int64_t ksb, kss, ksh;
  int B, S, H;
  const float *rope;
  int64_t rsb, rss;
  int rot;
  const uint16_t *qw, *kw;
  float eps;
  int64_t rows;  // B*S*H
};
int launch_qk_rmsnorm_rope(const RopeArgs &a, hipStream_t s);
// The same with the block means of the stored q and k (blocks of blk tokens)
// written to pq, pk [B,H,ceil(S/blk),128] fp32.
int launch_qk_rmsnorm_rope_pool(const RopeArgs &a, int blk, float *pq, float *pk, hipStream_t s);
int rope_kernel_attrs(double out[6]);

}  // namespace h3a
