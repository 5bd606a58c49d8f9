/*
 * h3_oracle.c - CPU restatement of the MiniMax-H3 attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker.  The product (libh3attn) never links or calls it.
 *
 * Functions and the reference behaviour each one restates (paths relative to
 * the reference checkout):
 *
 *  oracle_attn_fwd      - non-causal softmax(scale*QK^T)V, fp64 accumulation.
 *      attn_sm80/fa3_sm80_h3.cu:355-365  keys >= N masked out
 *      attn_sm80/fa3_sm80_h3.cu:377-394  softmax with row max and row sum of
 *                                        UNROUNDED p
 *      attn_sm80/fa3_sm80_h3.cu:405-420  P rounded to bf16 before PV (round_p=1)
 *      attn_sm80/fa3_sm80_h3.cu:443-457  O = acc / l, rows >= N not stored
 *      attn_sm80/bench_attn.py:22-24     oracle = SDPA, non-causal, scale 1/sqrt(D)
 *    An optional block map restricts query block i to the key blocks kept in
 *    map[i][*] (custom_nodes/h3_sla/__init__.py:226-235: skipped blocks
 *    contribute nothing); a query row with no kept key gets O = 0.
 *    The softmax uses the global row max (two passes), which is the exact
 *    value the reference's online rescaling converges to.
 *
 *  oracle_qk_rmsnorm_rope - in-place RMSNorm over head_dim with weight, then
 *      split-half RoPE with 2x2 rotation matrices (the call contract of
 *      comfy.quant_ops.ck.rms_rope_split_half_ at harness/sp_runtime.py:93-99
 *      and custom_nodes/h3_profiler/__init__.py:99-106; rot_dim =
 *      rope_freqs.shape[-3]*2).  comfy_kitchen is not vendored; its exact
 *      rounding is unknown, so this uses fp64 math and one bf16 rounding.
 *
 *  oracle_block_map     - mean-pool q and k over the valid rows of each block,
 *      score = pooled_q . pooled_k, keep the `keep` highest-scoring key blocks
 *      per query block (ties -> lower index), optionally force the diagonal
 *      block and optionally centre k by its mean over the sequence first
 *      (the block selection of SLA's get_block_map as used at
 *      custom_nodes/h3_sla/__init__.py:232; SLA is not vendored).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

float oracle_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round-to-nearest-even fp32 -> bf16 (NaN stays NaN). */
uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static double round_bf16(double x) { return (double)oracle_bf16_to_f32(oracle_f32_to_bf16((float)x)); }

/*
 * q: [B,H,Sq,D], k/v: [B,H,Skv,D] (bf16 bits, strides {b,h,s} in elements, d contiguous)
 * o: [B,H,Sq,D] fp32 with strides os.
 * block_map: NULL or uint8 [B,H,nq,nk] (contiguous), nq = ceil(Sq/blk_q), nk = ceil(Skv/blk_k).
 */
int oracle_attn_fwd(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *o, int B, int H,
                    int Sq, int Skv, int D, const int64_t *qs, const int64_t *ks, const int64_t *vs,
                    const int64_t *os, double scale, int round_p, const uint8_t *block_map,
                    int blk_q, int blk_k) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0 || D <= 0) return 1;
  const int nq = block_map ? (Sq + blk_q - 1) / blk_q : 0;
  const int nk = block_map ? (Skv + blk_k - 1) / blk_k : 0;
  int err = 0;
#pragma omp parallel
  {
    double *s = (double *)malloc(sizeof(double) * (size_t)Skv);
    double *acc = (double *)malloc(sizeof(double) * (size_t)D);
    float *qf = (float *)malloc(sizeof(float) * (size_t)D);
    if (!s || !acc || !qf) {
#pragma omp atomic write
      err = 2;
    }
    /* every thread reaches the worksharing loop; one without buffers skips rows */
#pragma omp for collapse(3) schedule(dynamic, 16)
      for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
          for (int i = 0; i < Sq; ++i) {
            if (!s || !acc || !qf) continue;
            const uint16_t *qr = q + b * qs[0] + h * qs[1] + (int64_t)i * qs[2];
            for (int d = 0; d < D; ++d) qf[d] = oracle_bf16_to_f32(qr[d]);
            const uint8_t *mrow = block_map ? block_map + (((int64_t)b * H + h) * nq + i / blk_q) * nk : NULL;
            double m = -INFINITY;
            for (int j = 0; j < Skv; ++j) {
              if (mrow && !mrow[j / blk_k]) {
                s[j] = -INFINITY;
                continue;
              }
              const uint16_t *kr = k + b * ks[0] + h * ks[1] + (int64_t)j * ks[2];
              double dot = 0.0;
              for (int d = 0; d < D; ++d) dot += (double)qf[d] * (double)oracle_bf16_to_f32(kr[d]);
              s[j] = dot * scale;
              if (s[j] > m) m = s[j];
            }
            for (int d = 0; d < D; ++d) acc[d] = 0.0;
            double l = 0.0;
            if (m > -INFINITY) {
              for (int j = 0; j < Skv; ++j) {
                if (s[j] == -INFINITY) continue;
                const double p = exp(s[j] - m);
                l += p;
                const double pv = round_p ? round_bf16(p) : p;
                const uint16_t *vr = v + b * vs[0] + h * vs[1] + (int64_t)j * vs[2];
                for (int d = 0; d < D; ++d) acc[d] += pv * (double)oracle_bf16_to_f32(vr[d]);
              }
            }
            float *orow = o + b * os[0] + h * os[1] + (int64_t)i * os[2];
            for (int d = 0; d < D; ++d) orow[d] = l > 0.0 ? (float)(acc[d] / l) : 0.0f;
          }
    free(s);
    free(acc);
    free(qf);
  }
  return err;
}

/*
 * In place on q, k: [B,S,H,D] bf16 with strides {b,s,h} (elements), d contiguous.
 * rope: fp32, element (b,s,i,r,c) at b*rsb + s*rss + i*4 + r*2 + c.
 * qw, kw: bf16 [D].
 */
int oracle_qk_rmsnorm_rope(uint16_t *q, uint16_t *k, int B, int S, int H, int D, const int64_t *qs,
                           const int64_t *ks, const float *rope, int64_t rsb, int64_t rss, int rot,
                           const uint16_t *qw, const uint16_t *kw, double eps) {
  if (B <= 0 || S <= 0 || H <= 0 || D <= 0 || D > 1024 || rot < 0 || rot > D || (rot & 1)) return 1;
  const int half = rot / 2;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int s = 0; s < S; ++s) {
      double y[1024];
      for (int t = 0; t < 2; ++t) {
        uint16_t *base = t == 0 ? q : k;
        const int64_t *st = t == 0 ? qs : ks;
        const uint16_t *w = t == 0 ? qw : kw;
        for (int h = 0; h < H; ++h) {
          uint16_t *x = base + b * st[0] + (int64_t)s * st[1] + h * st[2];
          double ss = 0.0;
          for (int d = 0; d < D; ++d) {
            const double xv = oracle_bf16_to_f32(x[d]);
            ss += xv * xv;
          }
          const double r = 1.0 / sqrt(ss / D + eps);
          for (int d = 0; d < D; ++d) y[d] = oracle_bf16_to_f32(x[d]) * r * oracle_bf16_to_f32(w[d]);
          for (int i = 0; i < half; ++i) {
            const float *R = rope + b * rsb + (int64_t)s * rss + (int64_t)i * 4;
            const double a = y[i], c = y[i + half];
            y[i] = (double)R[0] * a + (double)R[1] * c;
            y[i + half] = (double)R[2] * a + (double)R[3] * c;
          }
          for (int d = 0; d < D; ++d) x[d] = oracle_f32_to_bf16((float)y[d]);
        }
      }
    }
  return 0;
}

/*
 * Block map [B,H,nq,nk] (uint8 0/1, contiguous) from mean-pooled scores.
 * q: [B,H,Sq,D], k: [B,H,Skv,D] bf16 bits with strides {b,h,s}.
 * keep: key blocks kept per query block by score (clamped to [0,nk]).
 * scores_out: optional fp64 [B,H,nq,nk] pooled scores (after smoothing).
 */
int oracle_block_map(const uint16_t *q, const uint16_t *k, int B, int H, int Sq, int Skv, int D,
                     const int64_t *qs, const int64_t *ks, int blk_q, int blk_k, int keep,
                     int force_diag, int smooth_k, uint8_t *map, double *scores_out) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0 || D <= 0 || blk_q <= 0 || blk_k <= 0) return 1;
  const int nq = (Sq + blk_q - 1) / blk_q, nk = (Skv + blk_k - 1) / blk_k;
  if (keep < 0) keep = 0;
  if (keep > nk) keep = nk;
  int err = 0;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      double *pq = (double *)calloc((size_t)nq * D, sizeof(double));
      double *pk = (double *)calloc((size_t)nk * D, sizeof(double));
      double *kmean = (double *)calloc((size_t)D, sizeof(double));
      double *sc = (double *)malloc(sizeof(double) * (size_t)nk);
      char *taken = (char *)malloc((size_t)nk);
      if (!pq || !pk || !kmean || !sc || !taken) {
#pragma omp atomic write
        err = 2;
      } else {
        for (int i = 0; i < Sq; ++i) {
          const uint16_t *r = q + b * qs[0] + h * qs[1] + (int64_t)i * qs[2];
          for (int d = 0; d < D; ++d) pq[(i / blk_q) * D + d] += oracle_bf16_to_f32(r[d]);
        }
        for (int j = 0; j < Skv; ++j) {
          const uint16_t *r = k + b * ks[0] + h * ks[1] + (int64_t)j * ks[2];
          for (int d = 0; d < D; ++d) {
            const double x = oracle_bf16_to_f32(r[d]);
            pk[(j / blk_k) * D + d] += x;
            kmean[d] += x;
          }
        }
        for (int d = 0; d < D; ++d) kmean[d] /= Skv;
        for (int i = 0; i < nq; ++i) {
          const int cnt = (i + 1) * blk_q <= Sq ? blk_q : Sq - i * blk_q;
          for (int d = 0; d < D; ++d) pq[i * D + d] /= cnt;
        }
        for (int j = 0; j < nk; ++j) {
          const int cnt = (j + 1) * blk_k <= Skv ? blk_k : Skv - j * blk_k;
          for (int d = 0; d < D; ++d) {
            pk[j * D + d] /= cnt;
            if (smooth_k) pk[j * D + d] -= kmean[d];
          }
        }
        for (int i = 0; i < nq; ++i) {
          uint8_t *mrow = map + (((int64_t)b * H + h) * nq + i) * nk;
          for (int j = 0; j < nk; ++j) {
            double dot = 0.0;
            for (int d = 0; d < D; ++d) dot += pq[i * D + d] * pk[j * D + d];
            sc[j] = dot;
            mrow[j] = 0;
            taken[j] = 0;
            if (scores_out) scores_out[(((int64_t)b * H + h) * nq + i) * nk + j] = dot;
          }
          for (int t = 0; t < keep; ++t) {
            int best = -1;
            for (int j = 0; j < nk; ++j)
              if (!taken[j] && (best < 0 || sc[j] > sc[best])) best = j;
            taken[best] = 1;
            mrow[best] = 1;
          }
          if (force_diag) {
            const int jd = (int)(((int64_t)i * blk_q) / blk_k);
            if (jd < nk) mrow[jd] = 1;
          }
        }
      }
      free(pq);
      free(pk);
      free(kmean);
      free(sc);
      free(taken);
    }
  return err;
}
