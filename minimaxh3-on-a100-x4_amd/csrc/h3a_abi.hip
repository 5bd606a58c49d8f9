// extern "C" entry points of libh3attn (declared in include/h3attn.h):
// argument validation, error reporting, dispatch to the kernel launchers.
// Validation runs before any HIP call, so a bad argument never reaches the GPU.
#include <atomic>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "h3a_internal.h"

#ifdef H3A_PROFILE
#define H3A_PROFILE_BUILD (H3A_PROFILE != 0)
#else
#define H3A_PROFILE_BUILD 0
#endif

namespace h3a {

static thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = '\0'; }

int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(H3A_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return H3A_OK;
}

namespace {

constexpr int64_t kMaxSeqStride = int64_t(1) << 24;
constexpr int64_t kRowElems = 128;  // elements of one q/k/v/o row (head_dim)

bool strides_ok(const int64_t s[3]) {
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || (s[i] & 7) != 0) return false;
  return true;
}

// Checks shared by the dense and block-sparse attention entry points.
int check_attn(const void *q, const void *k, const void *v, void *o, int B, int H, int Sq, int Skv,
               int D, const int64_t *qs, const int64_t *ks, const int64_t *vs, const int64_t *os,
               float scale) {
  if (!q || !k || !v || !o) return fail(H3A_ERR_INVALID_ARG, "null tensor pointer");
  if (!qs || !ks || !vs || !os) return fail(H3A_ERR_INVALID_ARG, "null stride array");
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0)
    return fail(H3A_ERR_INVALID_ARG, "sizes must be positive (B=%d H=%d Sq=%d Skv=%d)", B, H, Sq, Skv);
  if (D != 128) return fail(H3A_ERR_UNSUPPORTED, "head_dim %d unsupported (only 128)", D);
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(H3A_ERR_INVALID_ARG, "softmax scale must be finite and > 0");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(H3A_ERR_ALIGNMENT, "tensor base pointers must be 16-byte aligned");
  if (!strides_ok(qs) || !strides_ok(ks) || !strides_ok(vs) || !strides_ok(os))
    return fail(H3A_ERR_ALIGNMENT, "strides must be non-negative multiples of 8 elements");
  if (Skv > INT_MAX - 256 || Sq > INT_MAX - 256) return fail(H3A_ERR_INVALID_ARG, "sequence too long");
  // A 64-key stage of K or V is addressed with 32-bit byte offsets from the
  // stage's first row (buffer range and per-lane offsets): 64 rows must span
  // less than 2 GiB.
  if (ks[2] >= kMaxSeqStride || vs[2] >= kMaxSeqStride)
    return fail(H3A_ERR_UNSUPPORTED, "k/v sequence stride must be < %lld elements", (long long)kMaxSeqStride);
  // Output rows closer than one row apart would overlap.  (A length-1
  // sequence has no second row: its stride is free, see fill_attn_args.)
  if (Sq > 1 && os[2] < kRowElems)
    return fail(H3A_ERR_INVALID_ARG, "o sequence stride %lld is less than a row (%lld elements): rows overlap",
                (long long)os[2], (long long)kRowElems);
  return H3A_OK;
}

// Scratch of the allocation-free dense entry point (h3a_attn_fwd_noalloc): the
// split-tail partials, (O row, m, l) in fp32 for each of the r * P key ranges
// of the last round's tiles, then 1 KiB of work-queue counters.  r * P <= CUs
// (P = CUs / r at most), so on a 256-CU device no plan needs more than
// 256 * 256 * (128 + 2) floats + 1 KiB.  Each GPU
// holds its own copy until the process ends.  In host code `scratch` only
// names the symbol; its device address comes from hipGetSymbolAddress, once per
// device (scratch_ptr).
constexpr size_t kScratchBytes = H3A_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes == (size_t)256 * 256 * (128 + 2) * sizeof(float) + 1024,
              "256-CU split tail, then the dense work queues' counters");
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's copy of `scratch`.
int scratch_ptr(void **out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(H3A_ERR_HIP, "hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return fail(H3A_ERR_UNSUPPORTED, "device index %d out of range", dev);
  void *p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p)
        return fail(H3A_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return H3A_OK;
}

void fill_attn_args(AttnArgs &a, const void *q, const void *k, const void *v, void *o, int B, int H,
                    int Sq, int Skv, const int64_t *qs, const int64_t *ks, const int64_t *vs,
                    const int64_t *os, float scale) {
  a.q = static_cast<const uint16_t *>(q);
  a.k = static_cast<const uint16_t *>(k);
  a.v = static_cast<const uint16_t *>(v);
  a.o = static_cast<uint16_t *>(o);
  a.qsb = qs[0]; a.qsh = qs[1]; a.qss = qs[2];
  a.ksb = ks[0]; a.ksh = ks[1]; a.kss = ks[2];
  a.vsb = vs[0]; a.vsh = vs[1]; a.vss = vs[2];
  a.osb = os[0]; a.osh = os[1]; a.oss = os[2];
  // The kernels step along the sequence past its end (whole 32-row O tiles,
  // 64-row K/V stages) and rely on a buffer range to drop those rows, which
  // takes a stride of at least one row.  A length-1 sequence's stride never
  // reaches a valid row, so callers may pass anything there (0 for a size-1
  // dimension, as torch views do): give it one row.
  if (Sq == 1) a.qss = a.oss = kRowElems;
  if (Skv == 1) a.kss = a.vss = kRowElems;
  a.B = B; a.H = H; a.Sq = Sq; a.Skv = Skv;
  a.sl2 = scale * 1.4426950408889634f;
  a.lut = nullptr; a.counts = nullptr; a.lut_stride = 0; a.sub = 1; a.blk_k = 64;
  a.nkb = 0; a.nqb = 0; a.qmul = 1;
  a.split_first = INT_MAX; a.split_pieces = 1; a.ws = nullptr; a.sched = nullptr; a.pair_map = nullptr;
}

}  // namespace
}  // namespace h3a

using namespace h3a;

extern "C" {

const char *h3a_version(void) { return "h3attn 0.1.0 gfx950"; }

const char *h3a_last_error(void) { return g_err; }

int h3a_attn_fwd(const void *q, const void *k, const void *v, void *o, int B, int H, int Sq, int Skv,
                 int D, const int64_t q_strides[3], const int64_t k_strides[3],
                 const int64_t v_strides[3], const int64_t o_strides[3], float scale,
                 h3a_stream_t stream) {
  clear_error();
  int rc = check_attn(q, k, v, o, B, H, Sq, Skv, D, q_strides, k_strides, v_strides, o_strides, scale);
  if (rc) return rc;
  AttnArgs a;
  fill_attn_args(a, q, k, v, o, B, H, Sq, Skv, q_strides, k_strides, v_strides, o_strides, scale);
  return launch_attn_dense(a, as_stream(stream));
}

int h3a_attn_fwd_noalloc(const void *q, const void *k, const void *v, void *o, int B, int H, int Sq,
                         int Skv, int D, const int64_t q_strides[3], const int64_t k_strides[3],
                         const int64_t v_strides[3], const int64_t o_strides[3], float scale,
                         h3a_stream_t stream) {
  clear_error();
  int rc = check_attn(q, k, v, o, B, H, Sq, Skv, D, q_strides, k_strides, v_strides, o_strides, scale);
  if (rc) return rc;
  SplitPlan plan;
  rc = plan_attn_split(B, H, Sq, Skv, &plan);
  if (rc) return rc;
  void *ws = nullptr;
  if (plan.bytes > 0) {
    if (plan.bytes > kScratchBytes)
      return fail(H3A_ERR_UNSUPPORTED, "split tail and queues need %zu bytes of scratch; the static array holds %zu",
                  plan.bytes, kScratchBytes);
    rc = scratch_ptr(&ws);
    if (rc) return rc;
  }
  AttnArgs a;
  fill_attn_args(a, q, k, v, o, B, H, Sq, Skv, q_strides, k_strides, v_strides, o_strides, scale);
  return launch_attn_dense_split(a, plan, ws, as_stream(stream));
}

int h3a_attn_fwd_workspace_size(int B, int H, int Sq, int Skv, int D, size_t *bytes) {
  clear_error();
  if (!bytes) return fail(H3A_ERR_INVALID_ARG, "null output pointer");
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0)
    return fail(H3A_ERR_INVALID_ARG, "sizes must be positive (B=%d H=%d Sq=%d Skv=%d)", B, H, Sq, Skv);
  if (D != 128) return fail(H3A_ERR_UNSUPPORTED, "head_dim %d unsupported (only 128)", D);
  SplitPlan plan;
  const int rc = plan_attn_split(B, H, Sq, Skv, &plan);
  if (rc) return rc;
  *bytes = plan.bytes;
  return H3A_OK;
}

int h3a_attn_fwd_ws(const void *q, const void *k, const void *v, void *o, int B, int H, int Sq, int Skv,
                    int D, const int64_t q_strides[3], const int64_t k_strides[3],
                    const int64_t v_strides[3], const int64_t o_strides[3], float scale,
                    void *workspace, size_t workspace_bytes, h3a_stream_t stream) {
  clear_error();
  int rc = check_attn(q, k, v, o, B, H, Sq, Skv, D, q_strides, k_strides, v_strides, o_strides, scale);
  if (rc) return rc;
  SplitPlan plan;
  rc = plan_attn_split(B, H, Sq, Skv, &plan);
  if (rc) return rc;
  if (plan.bytes > 0) {
    if (!workspace || workspace_bytes < plan.bytes)
      return fail(H3A_ERR_INVALID_ARG, "workspace of %zu bytes needed, %zu given", plan.bytes,
                  workspace ? workspace_bytes : (size_t)0);
    if (!aligned16(workspace)) return fail(H3A_ERR_ALIGNMENT, "workspace must be 16-byte aligned");
  }
  AttnArgs a;
  fill_attn_args(a, q, k, v, o, B, H, Sq, Skv, q_strides, k_strides, v_strides, o_strides, scale);
  return launch_attn_dense_split(a, plan, workspace, as_stream(stream));
}

namespace {

int check_blocks(int blk_q, int blk_k) {
  if (!sparse_block_ok(blk_q)) return fail(H3A_ERR_UNSUPPORTED, "blk_q %d unsupported (64, 128, 192 or 256)", blk_q);
  if (!sparse_block_ok(blk_k)) return fail(H3A_ERR_UNSUPPORTED, "blk_k %d unsupported (64, 128, 192 or 256)", blk_k);
  return H3A_OK;
}

// Checks shared by the block-sparse entry points; fills `a` on success.
int prepare_blocksparse(AttnArgs &a, const void *q, const void *k, const void *v, void *o, int B, int H,
                        int Sq, int Skv, int D, const int64_t q_strides[3], const int64_t k_strides[3],
                        const int64_t v_strides[3], const int64_t o_strides[3], const int32_t *lut,
                        const int32_t *counts, int blk_q, int blk_k, int max_k_blocks, float scale) {
  int rc = check_attn(q, k, v, o, B, H, Sq, Skv, D, q_strides, k_strides, v_strides, o_strides, scale);
  if (rc) return rc;
  if (!lut || !counts) return fail(H3A_ERR_INVALID_ARG, "null lut/counts pointer");
  rc = check_blocks(blk_q, blk_k);
  if (rc) return rc;
  const int64_t nkb = (Skv + blk_k - 1) / blk_k;
  if (max_k_blocks <= 0 || max_k_blocks > nkb)
    return fail(H3A_ERR_INVALID_ARG, "max_k_blocks %d outside [1, %lld]", max_k_blocks, (long long)nkb);
  const int rows = sparse_sub_block_rows(blk_q);
  const int64_t nsub = (Sq + rows - 1) / rows;
  const int64_t total = (int64_t)B * H * nsub;
  if (total > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "too many query tiles (%lld)", (long long)total);
  fill_attn_args(a, q, k, v, o, B, H, Sq, Skv, q_strides, k_strides, v_strides, o_strides, scale);
  a.nqt = (int)nsub;
  a.total = (int)total;
  a.lut = lut;
  a.counts = counts;
  a.lut_stride = max_k_blocks;
  a.blk_k = blk_k;
  a.sub = blk_k / 64;
  a.nkb = (int)nkb;
  a.nqb = (int)((Sq + blk_q - 1) / blk_q);
  a.qmul = blk_q / rows;
  return H3A_OK;
}

}  // namespace

int h3a_attn_fwd_blocksparse(const void *q, const void *k, const void *v, void *o, int B, int H,
                             int Sq, int Skv, int D, const int64_t q_strides[3],
                             const int64_t k_strides[3], const int64_t v_strides[3],
                             const int64_t o_strides[3], const int32_t *lut, const int32_t *counts,
                             int blk_q, int blk_k, int max_k_blocks, float scale,
                             h3a_stream_t stream) {
  clear_error();
  AttnArgs a;
  const int rc = prepare_blocksparse(a, q, k, v, o, B, H, Sq, Skv, D, q_strides, k_strides, v_strides,
                                     o_strides, lut, counts, blk_q, blk_k, max_k_blocks, scale);
  if (rc) return rc;
  return launch_attn_sparse(a, blk_q, as_stream(stream));
}

int h3a_attn_fwd_blocksparse_workspace_size(int B, int H, int Sq, int Skv, int D, int blk_q, int blk_k,
                                            int max_k_blocks, size_t *bytes) {
  clear_error();
  if (!bytes) return fail(H3A_ERR_INVALID_ARG, "null output pointer");
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0)
    return fail(H3A_ERR_INVALID_ARG, "sizes must be positive (B=%d H=%d Sq=%d Skv=%d)", B, H, Sq, Skv);
  if (D != 128) return fail(H3A_ERR_UNSUPPORTED, "head_dim %d unsupported (only 128)", D);
  int rc = check_blocks(blk_q, blk_k);
  if (rc) return rc;
  const int64_t nkb = (Skv + blk_k - 1) / blk_k;
  if (max_k_blocks <= 0 || max_k_blocks > nkb)
    return fail(H3A_ERR_INVALID_ARG, "max_k_blocks %d outside [1, %lld]", max_k_blocks, (long long)nkb);
  SplitPlan plan;
  rc = plan_attn_sparse_split(B, H, Sq, blk_q, blk_k, max_k_blocks, &plan);
  if (rc) return rc;
  *bytes = plan.bytes;
  return H3A_OK;
}

int h3a_attn_fwd_blocksparse_ws(const void *q, const void *k, const void *v, void *o, int B, int H,
                                int Sq, int Skv, int D, const int64_t q_strides[3],
                                const int64_t k_strides[3], const int64_t v_strides[3],
                                const int64_t o_strides[3], const int32_t *lut, const int32_t *counts,
                                int blk_q, int blk_k, int max_k_blocks, float scale, void *workspace,
                                size_t workspace_bytes, h3a_stream_t stream) {
  clear_error();
  AttnArgs a;
  int rc = prepare_blocksparse(a, q, k, v, o, B, H, Sq, Skv, D, q_strides, k_strides, v_strides, o_strides,
                               lut, counts, blk_q, blk_k, max_k_blocks, scale);
  if (rc) return rc;
  SplitPlan plan;
  rc = plan_attn_sparse_split(B, H, Sq, blk_q, blk_k, max_k_blocks, &plan);
  if (rc) return rc;
  if (plan.bytes > 0) {
    if (!workspace || workspace_bytes < plan.bytes)
      return fail(H3A_ERR_INVALID_ARG, "workspace of %zu bytes needed, %zu given", plan.bytes,
                  workspace ? workspace_bytes : (size_t)0);
    if (!aligned16(workspace)) return fail(H3A_ERR_ALIGNMENT, "workspace must be 16-byte aligned");
  }
  return launch_attn_sparse_split(a, blk_q, plan, workspace, as_stream(stream));
}

namespace {

// Checks shared by the tile-LUT entry points; fills `a` on success.
int prepare_tiles(AttnArgs &a, const void *q, const void *k, const void *v, void *o, int B, int H, int Sq,
                  int Skv, int D, const int64_t q_strides[3], const int64_t k_strides[3],
                  const int64_t v_strides[3], const int64_t o_strides[3], const int32_t *lut,
                  const int32_t *counts, int max_tiles, float scale) {
  int rc = check_attn(q, k, v, o, B, H, Sq, Skv, D, q_strides, k_strides, v_strides, o_strides, scale);
  if (rc) return rc;
  if (!lut || !counts) return fail(H3A_ERR_INVALID_ARG, "null tile_lut/tile_counts pointer");
  const int64_t ncols = ((int64_t)Skv + 31) / 32;
  if (ncols > kMaxTileColumns)
    return fail(H3A_ERR_UNSUPPORTED, "Skv %d past the tile LUT's %d columns of 32 keys", Skv, kMaxTileColumns);
  if (max_tiles <= 0 || max_tiles > ncols)
    return fail(H3A_ERR_INVALID_ARG, "max_tiles %d outside [1, %lld]", max_tiles, (long long)ncols);
  const int64_t nsub = ((int64_t)Sq + 63) / 64;
  const int64_t total = (int64_t)B * H * nsub;
  if (total > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "too many query tiles (%lld)", (long long)total);
  fill_attn_args(a, q, k, v, o, B, H, Sq, Skv, q_strides, k_strides, v_strides, o_strides, scale);
  a.nqt = (int)nsub;
  a.total = (int)total;
  a.lut = lut;
  a.counts = counts;
  a.lut_stride = max_tiles;
  a.blk_k = 32;  // a LUT entry names one 32-key column
  a.sub = 1;
  a.nkb = (int)ncols;
  a.nqb = (int)nsub;
  a.qmul = 1;
  return H3A_OK;
}

}  // namespace

int h3a_attn_fwd_blocksparse_tiles(const void *q, const void *k, const void *v, void *o, int B, int H, int Sq,
                                   int Skv, int D, const int64_t q_strides[3], const int64_t k_strides[3],
                                   const int64_t v_strides[3], const int64_t o_strides[3],
                                   const int32_t *tile_lut, const int32_t *tile_counts, int max_tiles, float scale,
                                   h3a_stream_t stream) {
  clear_error();
  AttnArgs a;
  const int rc = prepare_tiles(a, q, k, v, o, B, H, Sq, Skv, D, q_strides, k_strides, v_strides, o_strides,
                               tile_lut, tile_counts, max_tiles, scale);
  if (rc) return rc;
  return launch_attn_sparse(a, 64, as_stream(stream), true);
}

int h3a_attn_fwd_blocksparse_tiles_workspace_size(int B, int H, int Sq, int Skv, int D, int max_tiles,
                                                  size_t *bytes) {
  clear_error();
  if (!bytes) return fail(H3A_ERR_INVALID_ARG, "null output pointer");
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0)
    return fail(H3A_ERR_INVALID_ARG, "sizes must be positive (B=%d H=%d Sq=%d Skv=%d)", B, H, Sq, Skv);
  if (D != 128) return fail(H3A_ERR_UNSUPPORTED, "head_dim %d unsupported (only 128)", D);
  const int64_t ncols = ((int64_t)Skv + 31) / 32;
  if (ncols > kMaxTileColumns)
    return fail(H3A_ERR_UNSUPPORTED, "Skv %d past the tile LUT's %d columns of 32 keys", Skv, kMaxTileColumns);
  if (max_tiles <= 0 || max_tiles > ncols)
    return fail(H3A_ERR_INVALID_ARG, "max_tiles %d outside [1, %lld]", max_tiles, (long long)ncols);
  SplitPlan plan;
  const int rc = plan_attn_sparse_tiles(B, H, Sq, max_tiles, &plan);
  if (rc) return rc;
  *bytes = plan.bytes;
  return H3A_OK;
}

int h3a_attn_fwd_blocksparse_tiles_ws(const void *q, const void *k, const void *v, void *o, int B, int H, int Sq,
                                      int Skv, int D, const int64_t q_strides[3], const int64_t k_strides[3],
                                      const int64_t v_strides[3], const int64_t o_strides[3],
                                      const int32_t *tile_lut, const int32_t *tile_counts, int max_tiles,
                                      float scale, void *workspace, size_t workspace_bytes, h3a_stream_t stream) {
  clear_error();
  AttnArgs a;
  int rc = prepare_tiles(a, q, k, v, o, B, H, Sq, Skv, D, q_strides, k_strides, v_strides, o_strides, tile_lut,
                         tile_counts, max_tiles, scale);
  if (rc) return rc;
  SplitPlan plan;
  rc = plan_attn_sparse_tiles(B, H, Sq, max_tiles, &plan);
  if (rc) return rc;
  if (plan.bytes > 0) {
    if (!workspace || workspace_bytes < plan.bytes)
      return fail(H3A_ERR_INVALID_ARG, "workspace of %zu bytes needed, %zu given", plan.bytes,
                  workspace ? workspace_bytes : (size_t)0);
    if (!aligned16(workspace)) return fail(H3A_ERR_ALIGNMENT, "workspace must be 16-byte aligned");
  }
  return launch_attn_sparse_split(a, 64, plan, workspace, as_stream(stream), true);
}

int h3a_block_map_to_tile_lut(const uint8_t *block_map, int B, int H, int Sq, int Skv, int blk_q, int blk_k,
                              int32_t *tile_lut, int32_t *tile_counts, int max_tiles, h3a_stream_t stream) {
  clear_error();
  if (!block_map || !tile_lut || !tile_counts) return fail(H3A_ERR_INVALID_ARG, "null pointer");
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0)
    return fail(H3A_ERR_INVALID_ARG, "sizes must be positive (B=%d H=%d Sq=%d Skv=%d)", B, H, Sq, Skv);
  if (!tile_block_ok(blk_q) || !tile_block_ok(blk_k))
    return fail(H3A_ERR_UNSUPPORTED, "block sizes %d x %d: multiples of 16 only", blk_q, blk_k);
  const int64_t ncols = ((int64_t)Skv + 31) / 32;
  if (ncols > kMaxTileColumns)
    return fail(H3A_ERR_UNSUPPORTED, "Skv %d past the tile LUT's %d columns of 32 keys", Skv, kMaxTileColumns);
  if (max_tiles <= 0 || max_tiles > ncols)
    return fail(H3A_ERR_INVALID_ARG, "max_tiles %d outside [1, %lld]", max_tiles, (long long)ncols);
  const int64_t rows = (int64_t)B * H * ((Sq + 63) / 64);
  if ((rows + 3) / 4 > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "too many tile LUT rows");
  return launch_block_map_to_tile_lut(block_map, B, H, Sq, Skv, blk_q, blk_k, tile_lut, tile_counts, max_tiles,
                                      as_stream(stream));
}

int h3a_lut_to_block_map(const int32_t *lut, const int32_t *counts, int B, int H, int nq, int nk,
                         int max_k_blocks, uint8_t *block_map, h3a_stream_t stream) {
  clear_error();
  if (!lut || !counts || !block_map) return fail(H3A_ERR_INVALID_ARG, "null pointer");
  if (B <= 0 || H <= 0 || nq <= 0 || nk <= 0 || max_k_blocks <= 0)
    return fail(H3A_ERR_INVALID_ARG, "sizes must be positive (B=%d H=%d nq=%d nk=%d max_k_blocks=%d)", B, H, nq,
                nk, max_k_blocks);
  const int64_t rows = (int64_t)B * H * nq;
  if ((rows + 3) / 4 > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "block map too large");
  return launch_lut_to_block_map(lut, counts, B, H, nq, nk, max_k_blocks, block_map, as_stream(stream));
}

int h3a_block_map_to_lut(const uint8_t *block_map, int B, int H, int nq, int nk, int32_t *lut,
                         int32_t *counts, int max_k_blocks, h3a_stream_t stream) {
  clear_error();
  if (!block_map || !lut || !counts) return fail(H3A_ERR_INVALID_ARG, "null pointer");
  if (B <= 0 || H <= 0 || nq <= 0 || nk <= 0)
    return fail(H3A_ERR_INVALID_ARG, "sizes must be positive (B=%d H=%d nq=%d nk=%d)", B, H, nq, nk);
  if (max_k_blocks <= 0 || max_k_blocks > nk)
    return fail(H3A_ERR_INVALID_ARG, "max_k_blocks %d outside [1, %d]", max_k_blocks, nk);
  const int64_t rows = (int64_t)B * H * nq;
  if ((rows + 255) / 256 > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "block map too large");
  return launch_block_map_to_lut(block_map, B, H, nq, nk, lut, counts, max_k_blocks, as_stream(stream));
}

int h3a_block_pool(const void *x, int B, int H, int S, int D, const int64_t strides[3], int blk,
                   float *out, h3a_stream_t stream) {
  clear_error();
  if (!x || !out || !strides) return fail(H3A_ERR_INVALID_ARG, "null pointer");
  if (B <= 0 || H <= 0 || S <= 0 || blk <= 0)
    return fail(H3A_ERR_INVALID_ARG, "sizes must be positive (B=%d H=%d S=%d blk=%d)", B, H, S, blk);
  if (D != 128) return fail(H3A_ERR_UNSUPPORTED, "head_dim %d unsupported (only 128)", D);
  if (!aligned16(x) || !aligned16(out)) return fail(H3A_ERR_ALIGNMENT, "pointers must be 16-byte aligned");
  if (!strides_ok(strides)) return fail(H3A_ERR_ALIGNMENT, "strides must be non-negative multiples of 8 elements");
  const int64_t items = (int64_t)B * H * ((S + blk - 1) / blk);
  if ((items + 3) / 4 > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "too many blocks");
  return launch_block_pool(static_cast<const uint16_t *>(x), strides, B, H, S, blk, out, as_stream(stream));
}

int h3a_block_select(const float *pq, const float *pk, int B, int H, int nq, int nk, int keep,
                     int force_diag, int blk_q, int blk_k, int32_t *lut, int32_t *counts,
                     int max_k_blocks, uint8_t *block_map, h3a_stream_t stream) {
  clear_error();
  if (!pq || !pk || !lut || !counts) return fail(H3A_ERR_INVALID_ARG, "null pointer");
  if (B <= 0 || H <= 0 || nq <= 0 || nk <= 0 || blk_q <= 0 || blk_k <= 0)
    return fail(H3A_ERR_INVALID_ARG, "sizes must be positive");
  if (nk > 7000) return fail(H3A_ERR_UNSUPPORTED, "nk %d too large (max 7000 key blocks)", nk);
  if (keep < 0 || keep > nk) return fail(H3A_ERR_INVALID_ARG, "keep %d outside [0, %d]", keep, nk);
  if (max_k_blocks <= 0 || max_k_blocks > nk)
    return fail(H3A_ERR_INVALID_ARG, "max_k_blocks %d outside [1, %d]", max_k_blocks, nk);
  if (!aligned16(pq) || !aligned16(pk)) return fail(H3A_ERR_ALIGNMENT, "pq/pk must be 16-byte aligned");
  if ((int64_t)B * H * nq > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "too many query blocks");
  return launch_block_select(pq, pk, B, H, nq, nk, keep, force_diag ? 1 : 0, blk_q, blk_k, lut, counts,
                             max_k_blocks, block_map, as_stream(stream));
}

namespace {

// Checks shared by the prologue entry points; fills `a` on success.
int prepare_rope(RopeArgs &a, void *q, void *k, int B, int S, int H, int D, const int64_t q_strides[3],
                 const int64_t k_strides[3], const float *rope, int64_t rope_sb, int64_t rope_ss, int rot_dim,
                 const void *qw, const void *kw, float eps) {
  if (!q || !k || !qw || !kw) return fail(H3A_ERR_INVALID_ARG, "null tensor pointer");
  if (!q_strides || !k_strides) return fail(H3A_ERR_INVALID_ARG, "null stride array");
  if (B <= 0 || S <= 0 || H <= 0)
    return fail(H3A_ERR_INVALID_ARG, "sizes must be positive (B=%d S=%d H=%d)", B, S, H);
  if (D != 128) return fail(H3A_ERR_UNSUPPORTED, "head_dim %d unsupported (only 128)", D);
  if (rot_dim < 0 || rot_dim > D || (rot_dim % 16) != 0)
    return fail(H3A_ERR_UNSUPPORTED, "rot_dim %d must be a multiple of 16 in [0, %d]", rot_dim, D);
  if (rot_dim > 0 && !rope) return fail(H3A_ERR_INVALID_ARG, "null rope table with rot_dim > 0");
  if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(H3A_ERR_INVALID_ARG, "eps must be finite and >= 0");
  if (!aligned16(q) || !aligned16(k) || !aligned16(qw) || !aligned16(kw) || (rope && !aligned16(rope)))
    return fail(H3A_ERR_ALIGNMENT, "pointers must be 16-byte aligned");
  if (!strides_ok(q_strides) || !strides_ok(k_strides))
    return fail(H3A_ERR_ALIGNMENT, "q/k strides must be non-negative multiples of 8 elements");
  if (rot_dim > 0 && (rope_sb < 0 || rope_ss < 0 || (rope_sb & 3) || (rope_ss & 3)))
    return fail(H3A_ERR_ALIGNMENT, "rope strides must be non-negative multiples of 4 floats");
  const int64_t rows = (int64_t)B * S * H;
  const int64_t items = (int64_t)B * S * ((H + 15) / 16);  // (token, 16-head chunk) work items
  if ((items + 3) / 4 > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "too many tokens");
  a.q = static_cast<uint16_t *>(q);
  a.k = static_cast<uint16_t *>(k);
  a.qsb = q_strides[0]; a.qss = q_strides[1]; a.qsh = q_strides[2];
  a.ksb = k_strides[0]; a.kss = k_strides[1]; a.ksh = k_strides[2];
  a.B = B; a.S = S; a.H = H;
  a.rope = rope; a.rsb = rope_sb; a.rss = rope_ss; a.rot = rot_dim;
  a.qw = static_cast<const uint16_t *>(qw);
  a.kw = static_cast<const uint16_t *>(kw);
  a.eps = eps;
  a.rows = rows;
  return H3A_OK;
}

}  // namespace

int h3a_qk_rmsnorm_rope(void *q, void *k, int B, int S, int H, int D, const int64_t q_strides[3],
                        const int64_t k_strides[3], const float *rope, int64_t rope_sb,
                        int64_t rope_ss, int rot_dim, const void *qw, const void *kw, float eps,
                        h3a_stream_t stream) {
  clear_error();
  RopeArgs a;
  const int rc = prepare_rope(a, q, k, B, S, H, D, q_strides, k_strides, rope, rope_sb, rope_ss, rot_dim, qw, kw,
                              eps);
  if (rc) return rc;
  return launch_qk_rmsnorm_rope(a, as_stream(stream));
}

int h3a_qk_rmsnorm_rope_pool(void *q, void *k, int B, int S, int H, int D, const int64_t q_strides[3],
                             const int64_t k_strides[3], const float *rope, int64_t rope_sb, int64_t rope_ss,
                             int rot_dim, const void *qw, const void *kw, float eps, int blk, float *q_means,
                             float *k_means, h3a_stream_t stream) {
  clear_error();
  RopeArgs a;
  const int rc = prepare_rope(a, q, k, B, S, H, D, q_strides, k_strides, rope, rope_sb, rope_ss, rot_dim, qw, kw,
                              eps);
  if (rc) return rc;
  if (!q_means || !k_means) return fail(H3A_ERR_INVALID_ARG, "null block-mean pointer");
  if (!aligned16(q_means) || !aligned16(k_means)) return fail(H3A_ERR_ALIGNMENT, "block means must be 16-byte aligned");
  if (blk <= 0) return fail(H3A_ERR_INVALID_ARG, "blk %d must be positive", blk);
  const int64_t wgs = (int64_t)B * ((S + blk - 1) / blk) * ((H + 7) / 8);
  if (wgs > INT_MAX) return fail(H3A_ERR_INVALID_ARG, "too many blocks");
  return launch_qk_rmsnorm_rope_pool(a, blk, q_means, k_means, as_stream(stream));
}

int h3a_kernel_attrs(int which, double out[6]) {
  clear_error();
  if (!out) return fail(H3A_ERR_INVALID_ARG, "null output array");
  if (which == H3A_KERNEL_QK_ROPE) return rope_kernel_attrs(out);
  if (which != H3A_KERNEL_ATTN_SPARSE_TILES && (which < H3A_KERNEL_ATTN_DENSE || which > H3A_KERNEL_ATTN_SPARSE_64))
    return fail(H3A_ERR_INVALID_ARG, "unknown kernel id %d", which);
  return attn_kernel_attrs(which, out);
}

int h3a_prof_enabled(void) { return H3A_PROFILE_BUILD; }

int h3a_prof_read(uint64_t out[H3A_PROF_WAVES * H3A_PROF_SLOTS]) {
  clear_error();
  if (!out) return fail(H3A_ERR_INVALID_ARG, "null output array");
  return attn_prof_read(out);
}

int h3a_prof_reset(void) {
  clear_error();
  return attn_prof_reset();
}

int h3a_test_qk(const void *Q, const void *K, float *S, h3a_stream_t stream) {
  clear_error();
  if (!Q || !K || !S) return fail(H3A_ERR_INVALID_ARG, "null pointer");
  if (!aligned16(Q) || !aligned16(K)) return fail(H3A_ERR_ALIGNMENT, "Q/K must be 16-byte aligned");
  return launch_test_qk(static_cast<const uint16_t *>(Q), static_cast<const uint16_t *>(K), S,
                        as_stream(stream));
}

int h3a_test_pv(const void *P, const void *V, float *O, h3a_stream_t stream) {
  clear_error();
  if (!P || !V || !O) return fail(H3A_ERR_INVALID_ARG, "null pointer");
  if (!aligned16(P) || !aligned16(V)) return fail(H3A_ERR_ALIGNMENT, "P/V must be 16-byte aligned");
  return launch_test_pv(static_cast<const uint16_t *>(P), static_cast<const uint16_t *>(V), O,
                        as_stream(stream));
}

}  // extern "C"
