/*
 * h3attn.h - C ABI of the MI355X (gfx950) exact-attention library for the
 * MiniMax-H3 video DiT: dense flash-attention forward, block-sparse forward,
 * fused per-head qk-RMSNorm + split-half RoPE prologue.
 *
 * Conventions (every entry point):
 *   - bf16 tensors are passed as raw device pointers (uint16_t storage).
 *   - Strides are in ELEMENTS; the innermost (head_dim) stride is always 1.
 *   - Device pointers and every outer stride must be 16-byte aligned
 *     (strides multiple of 8 elements) so rows move as 128-bit accesses.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream)
 *     and never synchronised.  Thread-safe: the only state shared between
 *     calls is (a) per-device caches of the CU count, occupancy and the
 *     scratch address, each set once and read atomically; (b) the static
 *     scratch array of h3a_attn_fwd_noalloc, one per GPU and shared by every
 *     call of that entry point on it, so such calls that overlap on one GPU
 *     race (see there); (c) in the profile build only, the phase-profile
 *     slots, which every launch of a ping-pong kernel overwrites
 *     (h3a_prof_read).
 *   - Return 0 (H3A_OK) on success, a non-zero H3A_ERR_* code otherwise;
 *     h3a_last_error() then holds a thread-local message.  Argument checks run
 *     before any HIP call, so bad arguments never reach the GPU.
 *
 * Reference surfaces replaced (paths relative to the reference checkout):
 *   attn_sm80/fa3_sm80_h3.cu:460-470  fa3_sm80_h3_launch  -> h3a_attn_fwd
 *   attn_sm80/fa3_sm80_h3.cu:472-482  fa3_pp_launch       -> h3a_attn_fwd
 *   attn_sm80/fa3_sm80_h3.cu:485-512  kernel_attrs/pp_attrs -> h3a_kernel_attrs
 *   attn_sm80/fa3_sm80_h3.cu:516-570  test_qk/test_pv     -> h3a_test_qk/h3a_test_pv
 *   attn_sm80/fa3_sm80_h3.cu:584-593  pybind module       -> this header
 *   custom_nodes/h3_sla/__init__.py:232-234 get_block_map + SLA _attention.apply
 *                                     -> h3a_block_map_to_lut + h3a_attn_fwd_blocksparse
 *   harness/sp_runtime.py:98, custom_nodes/h3_profiler/__init__.py:104-105
 *     comfy.quant_ops.ck.rms_rope_split_half_  -> h3a_qk_rmsnorm_rope
 */
#ifndef H3ATTN_H
#define H3ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define H3A_OK               0
#define H3A_ERR_INVALID_ARG  1  /* null pointer, non-positive size, bad value   */
#define H3A_ERR_UNSUPPORTED  2  /* head_dim != 128, unsupported tile size, ...  */
#define H3A_ERR_ALIGNMENT    3  /* pointer or stride not 16-byte aligned        */
#define H3A_ERR_HIP          4  /* a HIP runtime call or kernel launch failed   */

/* hipStream_t, kept opaque so FFI callers need no HIP headers. */
typedef void *h3a_stream_t;

/* Library version string, e.g. "h3attn 0.1.0 gfx950". */
const char *h3a_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char *h3a_last_error(void);

/*
 * Dense non-causal attention forward:
 *   O[b,h,i,:] = softmax_j(scale * Q[b,h,i,:] . K[b,h,j,:]) V[b,h,j,:]
 * q: [B,H,Sq,D], k/v: [B,H,Skv,D], o: [B,H,Sq,D], all bf16, D == 128.
 * *_strides = {batch, head, seq} in elements.  fp32 accumulation; P is
 * rounded to bf16 before the PV product (as the reference kernel does,
 * attn_sm80/fa3_sm80_h3.cu:405-420).  Sq != Skv is allowed (pad path,
 * harness/sp_runtime.py:106-109).  scale > 0 (1/sqrt(128) for the DiT).
 * The seq strides of k and v must be < 2^24 elements (H3A_ERR_UNSUPPORTED).
 * With Sq > 1 the seq stride of o must be at least D, so that rows do not
 * overlap (H3A_ERR_INVALID_ARG).  The seq stride of a length-1 sequence
 * (Sq or Skv == 1) is ignored, as for any size-1 dimension: 0 is fine.
 * Range: the softmax runs against a stale reference max that is refreshed
 * once a stage's p values would exceed 2^16, so the unnormalised fp32 O is
 * bounded by 2^17 * ceil(Skv/64) * max|v|; results are finite for
 * max|v| < 2^128 / (2^17 * ceil(Skv/64)), about 3.9e30 at Skv = 42120 (the
 * reference's max-subtracted softmax, with every p <= 1, stays finite up to
 * 2^128 / Skv, about 8e33 there).
 * Replaces fa3_sm80_h3_launch (attn_sm80/fa3_sm80_h3.cu:460-470), which
 * ignored B, fixed the scale and launched on the legacy default stream.
 */
int h3a_attn_fwd(const void *q, const void *k, const void *v, void *o,
                 int B, int H, int Sq, int Skv, int D,
                 const int64_t q_strides[3], const int64_t k_strides[3],
                 const int64_t v_strides[3], const int64_t o_strides[3],
                 float scale, h3a_stream_t stream);

/*
 * h3a_attn_fwd with a caller-supplied device workspace (no allocation in the
 * library).  With it, the query tiles of the last, partly filled round of
 * workgroups are split into key ranges that run side by side and are merged
 * by a second kernel on the same stream; results equal h3a_attn_fwd's within
 * floating-point rounding.  Problems of four or more rounds of tiles also
 * run on a persistent grid whose workgroups take tiles from per-XCD work
 * queues (1 KiB of counters in the workspace, cleared by the call itself
 * with a kernel before the attention launch).  h3a_attn_fwd_workspace_size
 * gives the bytes needed for a problem on the current device (0: nothing is
 * split or queued, and workspace may be NULL).  The workspace must stay untouched until the call's
 * work on `stream` has completed, and two calls in flight at once need two
 * workspaces.  Same arguments and errors as h3a_attn_fwd, plus
 * H3A_ERR_INVALID_ARG for a missing or short workspace.  This entry point has
 * no counterpart in the reference; h3a_attn_fwd is the drop-in for
 * fa3_sm80_h3_launch.
 */
int h3a_attn_fwd_workspace_size(int B, int H, int Sq, int Skv, int D, size_t *bytes);
int h3a_attn_fwd_ws(const void *q, const void *k, const void *v, void *o,
                    int B, int H, int Sq, int Skv, int D,
                    const int64_t q_strides[3], const int64_t k_strides[3],
                    const int64_t v_strides[3], const int64_t o_strides[3],
                    float scale, void *workspace, size_t workspace_bytes, h3a_stream_t stream);

/*
 * h3a_attn_fwd_ws without a workspace argument and without any allocation:
 * the split-tail partials and the work queues' counters go to a static device
 * array of H3A_NOALLOC_SCRATCH_BYTES (32.5 MiB + 1 KiB) that each GPU the library runs on holds
 * until the process ends.  No counterpart in the reference: it is for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It calls no hipMalloc/hipFree and no
 * allocating library routine.  Every call on a GPU shares that GPU's array, so
 * calls that overlap on one GPU (other streams, other threads) race: the
 * caller must serialise them.  Every byte the merge reads is written earlier
 * by the same call, and the call clears the queue counters itself (with a
 * kernel, not a memset), so nothing needs clearing between calls.  A split tail
 * larger than the array (a device with more than 256 CUs) gives
 * H3A_ERR_UNSUPPORTED.  Same kernels and split plan as h3a_attn_fwd_ws, so the
 * results are equal bit for bit; same arguments and errors as h3a_attn_fwd.
 */
#define H3A_NOALLOC_SCRATCH_BYTES 34079744u
int h3a_attn_fwd_noalloc(const void *q, const void *k, const void *v, void *o,
                         int B, int H, int Sq, int Skv, int D,
                         const int64_t q_strides[3], const int64_t k_strides[3],
                         const int64_t v_strides[3], const int64_t o_strides[3],
                         float scale, h3a_stream_t stream);

/*
 * Block-sparse attention forward (h3_sla path, custom_nodes/h3_sla/__init__.py:226-235).
 * Query block qb of (b,h) attends only to the key blocks listed in
 *   lut[((b*H + h)*nqb + qb)*max_k_blocks + 0 .. counts[(b*H+h)*nqb + qb]-1]
 * (key-block indices in units of blk_k keys; nqb = ceil(Sq/blk_q)).
 * Skipped blocks contribute nothing; a query block with no kept key block
 * gets O = 0.  LUT entries that name no key block (negative, or at or past
 * ceil(Skv/blk_k)) are skipped as well.  blk_q and blk_k each in
 * {64, 128, 192, 256} (multiples of the kernels' 64-key stage); the h3_sla
 * node's other sizes (multiples of 16 from 16 to 256,
 * custom_nodes/h3_sla/__init__.py:315) give H3A_ERR_UNSUPPORTED here and run
 * through h3a_attn_fwd_blocksparse_tiles.  Other arguments as h3a_attn_fwd.
 */
int h3a_attn_fwd_blocksparse(const void *q, const void *k, const void *v, void *o,
                             int B, int H, int Sq, int Skv, int D,
                             const int64_t q_strides[3], const int64_t k_strides[3],
                             const int64_t v_strides[3], const int64_t o_strides[3],
                             const int32_t *lut, const int32_t *counts,
                             int blk_q, int blk_k, int max_k_blocks,
                             float scale, h3a_stream_t stream);

/*
 * h3a_attn_fwd_blocksparse with a caller-supplied device workspace, as
 * h3a_attn_fwd_ws is to h3a_attn_fwd: with blk_q = 128, the pairs of query
 * blocks in the last, partly filled round of workgroups are each split into
 * ranges of their kept-block lists that run side by side, merged by a second
 * kernel on the same stream (results equal h3a_attn_fwd_blocksparse's within
 * floating-point rounding).  Problems of four or more rounds of pairs run on
 * a persistent grid fed by per-XCD work queues, as in h3a_attn_fwd_ws (1 KiB
 * of counters in the workspace, cleared by the call).
 * h3a_attn_fwd_blocksparse_workspace_size gives the bytes needed on the
 * current device (0: nothing is split or queued, and workspace may be NULL);
 * the workspace rules are those of h3a_attn_fwd_ws.  This entry
 * point has no counterpart in the reference; h3a_attn_fwd_blocksparse is the
 * drop-in for the h3_sla path.
 */
int h3a_attn_fwd_blocksparse_workspace_size(int B, int H, int Sq, int Skv, int D,
                                            int blk_q, int blk_k, int max_k_blocks, size_t *bytes);
int h3a_attn_fwd_blocksparse_ws(const void *q, const void *k, const void *v, void *o,
                                int B, int H, int Sq, int Skv, int D,
                                const int64_t q_strides[3], const int64_t k_strides[3],
                                const int64_t v_strides[3], const int64_t o_strides[3],
                                const int32_t *lut, const int32_t *counts,
                                int blk_q, int blk_k, int max_k_blocks,
                                float scale, void *workspace, size_t workspace_bytes,
                                h3a_stream_t stream);

/*
 * Block-sparse attention over 32-key columns with sub-block masks: the path
 * for block sizes h3a_attn_fwd_blocksparse does not take (the h3_sla node
 * offers every multiple of 16 from 16 to 256, custom_nodes/h3_sla/__init__.py:315;
 * query and key blocks may differ).  The tile LUT comes from
 * h3a_block_map_to_tile_lut: row (b*H + h)*ceil(Sq/64) + qs of tile_lut
 * [.., max_tiles] lists, for query rows 64*qs .. 64*qs+63, the 32-key columns
 * to attend to, ascending, each entry column << 8 | mask, where bit 2*i + j of
 * the mask admits rows 64*qs + 16*i .. +15 against keys 32*column + 16*j .. +15
 * (every other score of the column is masked); tile_counts holds each row's
 * length.  The kernel takes a row's columns two at a time.  Entries whose
 * column is negative or at or past ceil(Skv/32) load nothing.  A row with no
 * admitted key gets O = 0.  Skv <= 65534 * 32.  max_tiles in
 * [1, ceil(Skv/32)].  Other arguments as h3a_attn_fwd; _ws and
 * _workspace_size as for h3a_attn_fwd_blocksparse_ws (work queues, no split).
 * The kernel runs two rows (64-row sub-blocks) per workgroup for as many
 * stages as the longer of the two; h3a_attn_fwd_blocksparse_tiles pairs rows
 * 2p and 2p+1, the _ws variant pairs them by length (a kernel sorts each
 * (b,h)'s rows into the workspace first; up to ceil(Sq/64) = 16384, beyond
 * that as the plain call).  Results are the same bit for bit; the workspace
 * is never 0 bytes then.
 * No counterpart in the reference's own code: SLA's Triton kernel takes the
 * same block maps at these sizes.
 */
int h3a_attn_fwd_blocksparse_tiles(const void *q, const void *k, const void *v, void *o,
                                   int B, int H, int Sq, int Skv, int D,
                                   const int64_t q_strides[3], const int64_t k_strides[3],
                                   const int64_t v_strides[3], const int64_t o_strides[3],
                                   const int32_t *tile_lut, const int32_t *tile_counts, int max_tiles,
                                   float scale, h3a_stream_t stream);
int h3a_attn_fwd_blocksparse_tiles_workspace_size(int B, int H, int Sq, int Skv, int D, int max_tiles,
                                                  size_t *bytes);
int h3a_attn_fwd_blocksparse_tiles_ws(const void *q, const void *k, const void *v, void *o,
                                      int B, int H, int Sq, int Skv, int D,
                                      const int64_t q_strides[3], const int64_t k_strides[3],
                                      const int64_t v_strides[3], const int64_t o_strides[3],
                                      const int32_t *tile_lut, const int32_t *tile_counts, int max_tiles,
                                      float scale, void *workspace, size_t workspace_bytes,
                                      h3a_stream_t stream);

/*
 * Convert a 0/1 block map [B,H,ceil(Sq/blk_q),ceil(Skv/blk_k)] (uint8,
 * contiguous) at any block sizes that are multiples of 16 into the tile LUT of
 * h3a_attn_fwd_blocksparse_tiles: tile_lut [B,H,ceil(Sq/64),max_tiles] (-1
 * padded) and tile_counts [B,H,ceil(Sq/64)].  A row with more than max_tiles
 * columns keeps its first max_tiles; max_tiles = ceil(Skv/32) always suffices.
 * The SLA block map (custom_nodes/h3_sla/__init__.py:232) at the node's
 * block sizes.
 */
int h3a_block_map_to_tile_lut(const uint8_t *block_map, int B, int H, int Sq, int Skv, int blk_q, int blk_k,
                              int32_t *tile_lut, int32_t *tile_counts, int max_tiles, h3a_stream_t stream);

/*
 * The inverse of h3a_block_map_to_lut: block_map [B,H,nq,nk] (uint8) = 1 for
 * the key blocks each LUT row lists (its first counts[row] entries; entries
 * outside [0, nk) ignored), 0 elsewhere.  Two kernels on `stream`.  For
 * callers that hold an h3_sla LUT at a block size that runs through
 * h3a_attn_fwd_blocksparse_tiles.
 */
int h3a_lut_to_block_map(const int32_t *lut, const int32_t *counts, int B, int H, int nq, int nk,
                         int max_k_blocks, uint8_t *block_map, h3a_stream_t stream);

/*
 * Compact a boolean block map [B,H,nq,nk] (uint8, 0/1, contiguous) into the
 * LUT form h3a_attn_fwd_blocksparse consumes: lut [B,H,nq,max_k_blocks]
 * (kept key-block indices in ascending order, tail entries set to -1) and
 * counts [B,H,nq].  Rows with more than max_k_blocks kept blocks are an
 * error only if detected on the host; the device clamps to max_k_blocks.
 * Replaces the (sparse_map, lut) pair returned by SLA's get_block_map
 * (custom_nodes/h3_sla/__init__.py:232).
 */
int h3a_block_map_to_lut(const uint8_t *block_map, int B, int H, int nq, int nk,
                         int32_t *lut, int32_t *counts, int max_k_blocks,
                         h3a_stream_t stream);

/*
 * Block means for the block map: out[b,h,j,:] = mean of x[b,h,r,:] over the
 * valid rows r of block j (blocks of blk rows; the last may be partial).
 * x: bf16 [B,H,S,D] with strides {batch, head, seq} (elements), D == 128.
 * out: fp32 [B,H,ceil(S/blk),128], contiguous.  The pooling step of SLA's
 * get_block_map (custom_nodes/h3_sla/__init__.py:232).
 */
int h3a_block_pool(const void *x, int B, int H, int S, int D, const int64_t strides[3], int blk,
                   float *out, h3a_stream_t stream);

/*
 * Top-k block selection from pooled blocks: score(i,j) = pq[i] . pk[j]; query
 * block i keeps the `keep` highest-scoring key blocks (ties: lower index
 * first) plus, if force_diag, key block floor(i*blk_q/blk_k).  Writes the
 * kept indices ascending into lut [B,H,nq,max_k_blocks] (-1 padded), their
 * number into counts [B,H,nq], and, if block_map is not NULL, the 0/1 map
 * [B,H,nq,nk].  pq: fp32 [B,H,nq,128], pk: fp32 [B,H,nk,128], contiguous.
 * Scores are fp32 products and sums in the order of the fp32 matrix-core
 * instruction (not a sequential dot product), so a key block whose score ties
 * the keep-th one to the last bits may go either way; exact ties keep the
 * lower index.  nk <= 7000 (H3A_ERR_UNSUPPORTED beyond).
 * The selection step of SLA's get_block_map (custom_nodes/h3_sla/__init__.py:232).
 */
int h3a_block_select(const float *pq, const float *pk, int B, int H, int nq, int nk, int keep,
                     int force_diag, int blk_q, int blk_k, int32_t *lut, int32_t *counts,
                     int max_k_blocks, uint8_t *block_map, h3a_stream_t stream);

/*
 * Fused per-head qk-RMSNorm + split-half RoPE, in place on q and k
 * (comfy.quant_ops.ck.rms_rope_split_half_, called at harness/sp_runtime.py:98
 * and custom_nodes/h3_profiler/__init__.py:104-105).
 * q, k: [B,S,H,D] bf16 views; *_strides = {batch, seq, head} in elements
 * (the DiT passes strided views of the fused QKV output: seq stride 3*H*D).
 * For every (b,s,h) row x (fp32 math):
 *   y = x * rsqrt(mean(x^2) + eps) * w            (w = qw or kw, bf16 [D])
 *   for i < rot_dim/2, with R = rope[b,s,i] (2x2, row-major):
 *     y'[i]           = R00*y[i] + R01*y[i+rot_dim/2]
 *     y'[i+rot_dim/2] = R10*y[i] + R11*y[i+rot_dim/2]
 *   dims >= rot_dim are only normalised; result rounded to bf16 (RNE).
 * rope: fp32, element (b,s,i,r,c) at b*rope_sb + s*rope_ss + i*4 + r*2 + c
 * (ComfyUI's rope_freqs [B,S,1,rot/2,2,2] layout; rope_sb may be 0).
 * rot_dim: even, multiple of 16, <= D.  D == 128.
 */
int h3a_qk_rmsnorm_rope(void *q, void *k, int B, int S, int H, int D,
                        const int64_t q_strides[3], const int64_t k_strides[3],
                        const float *rope, int64_t rope_sb, int64_t rope_ss,
                        int rot_dim, const void *qw, const void *kw, float eps,
                        h3a_stream_t stream);

/*
 * h3a_qk_rmsnorm_rope with SLA's block pooling fused in: the same in-place
 * update of q and k, and the fp32 means of the stored (bf16) q and k over
 * blocks of blk tokens, q_means / k_means [B,H,ceil(S/blk),128] contiguous
 * (the last block's mean over its valid tokens), equal bit for bit to
 * h3a_block_pool on the updated q and k.  For a layer whose attention is
 * block-sparse: the pooling step of SLA's get_block_map
 * (custom_nodes/h3_sla/__init__.py:232) then needs no second pass over q and
 * k.  No counterpart in the reference's code.  blk > 0; other arguments and
 * errors as h3a_qk_rmsnorm_rope.
 */
int h3a_qk_rmsnorm_rope_pool(void *q, void *k, int B, int S, int H, int D,
                             const int64_t q_strides[3], const int64_t k_strides[3],
                             const float *rope, int64_t rope_sb, int64_t rope_ss,
                             int rot_dim, const void *qw, const void *kw, float eps,
                             int blk, float *q_means, float *k_means, h3a_stream_t stream);

/* Kernel identifiers for h3a_kernel_attrs. */
#define H3A_KERNEL_ATTN_DENSE      0
#define H3A_KERNEL_ATTN_SPARSE_128 1
#define H3A_KERNEL_ATTN_SPARSE_64  2
#define H3A_KERNEL_QK_ROPE         3
#define H3A_KERNEL_ATTN_SPARSE_TILES 4

/*
 * out[6] = {VGPRs per thread, LDS bytes per workgroup, max resident
 * workgroups per CU, device clock kHz, occupancy (resident waves / max
 * waves per CU), threads per workgroup}.  Mirrors kernel_attrs/pp_attrs
 * (attn_sm80/fa3_sm80_h3.cu:485-512).  Queries the current device.
 */
int h3a_kernel_attrs(int which, double out[6]);

/*
 * Phase profile of the dense kernel: the counterpart of the reference's
 * -DPROFILE build and its get_prof / reset_prof (attn_sm80/fa3_sm80_h3.cu:96-105,
 * 572-582).  Only the profile build of this library (libh3attn_prof.so, compiled
 * with H3A_PROFILE=1) records anything.  There, every dense launch of
 * h3a_attn_fwd / h3a_attn_fwd_ws has its workgroup 0 write, for each of its
 * H3A_PROF_WAVES waves, H3A_PROF_SLOTS values (row-major [wave][slot]):
 *   [0] DMA issue (and the loop's branch)  [1] first cluster  [2] mid-stage barrier
 *   [3] second cluster  [4] DMA wait  [5] end-of-stage barrier  [6] stages run
 *   [7] whole stage loop  [8] whole stage loop in 100 MHz ticks (s_memrealtime)
 *   [9] epilogue  [10] prologue  [11] 0
 * in shader-clock ticks (s_memtime) except [6] and [8]; [0]-[5] sum to [7].
 * Waves 0-3 run the matrix cluster (QK^T and PV MFMAs) first and the softmax
 * second, waves 4-7 the other way round.  A later launch overwrites the slots.
 *   h3a_prof_enabled: 1 in the profile build, 0 otherwise.
 *   h3a_prof_read:    synchronises the current device, copies the slots to out.
 *   h3a_prof_reset:   synchronises the current device, zeroes the slots.
 */
#define H3A_PROF_WAVES 8
#define H3A_PROF_SLOTS 12
int h3a_prof_enabled(void);
int h3a_prof_read(uint64_t out[H3A_PROF_WAVES * H3A_PROF_SLOTS]);
int h3a_prof_reset(void);

/*
 * Fragment tests on one wavefront through the same LDS staging and MFMA
 * fragment code as the attention kernel (counterparts of test_qk/test_pv,
 * attn_sm80/fa3_sm80_h3.cu:516-570):
 *   h3a_test_qk: S[32,64] (fp32) = Q[32,128] @ K[64,128]^T   (bf16 inputs)
 *   h3a_test_pv: O[32,128] (fp32) = P[32,64] @ V[64,128]     (bf16 inputs)
 * All buffers contiguous, row-major, device memory.
 */
int h3a_test_qk(const void *Q, const void *K, float *S, h3a_stream_t stream);
int h3a_test_pv(const void *P, const void *V, float *O, h3a_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* H3ATTN_H */
