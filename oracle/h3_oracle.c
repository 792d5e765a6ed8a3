/*
 * h3_oracle.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A CPU restatement of the reference's attention hot path. It is the checker
 * the HIP library is compared against and the CPU baseline bench.py times;
 * the product never calls into it. Citations are to the reference tree
 * (loading-awesome/MiniMax-H3-Swift).
 *
 * Pinning (what keeps this restatement honest) lives in tests/test_oracle_*.py:
 * closed-form tile counts, the reference's own known-answer tokens and
 * landmark sets, counted-vs-closed-form density, torch's fp32 SDPA as an
 * independent library, streaming-vs-masked and chunking invariance, and
 * rotation/normalisation invariants for the prologue.
 */
#include "h3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ bf16 */

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void orc_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(in[i]);
}

void orc_bf16_to_f32_n(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = orc_bf16_to_f32(in[i]);
}

static float rbf(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

/* -------------------------------------------------------------- topology */

/* AxialTopology.locate (Sources/H3Attention/AxialTopology.swift:115-120). */
static int locate(const orc_rule* r, int32_t tok, int32_t* f, int32_t* y, int32_t* x) {
  if (tok < r->prefix_len || tok >= r->seq_len) return 0;
  int32_t v = tok - r->prefix_len, per = r->height * r->width;
  *f = v / per;
  *y = (v % per) / r->width;
  *x = v % r->width;
  return 1;
}

static int is_landmark(const orc_rule* r, int32_t frame) {
  for (int32_t i = 0; i < r->n_landmarks; i++)
    if (r->landmarks[i] == frame) return 1;
  return 0;
}

/* Per-pair predicate. AXIAL is AxialTopology.allows
 * (AxialTopology.swift:128-137). LOCAL is the written local-window rule for
 * the synthetic benchmark shapes: prefix rows and columns dense, otherwise
 * |dt| <= frame_window and the two tokens' spatial tiles within sp_window on
 * both axes, plus any landmark frame. BAND is defined on tiles, so it is
 * evaluated on (q/tile, k/tile). */
int orc_allows(const orc_rule* r, int32_t q, int32_t k) {
  if (q < 0 || k < 0 || q >= r->seq_len || k >= r->seq_len) return 0;
  switch (r->kind) {
    case ORC_RULE_DENSE:
      return 1;
    case ORC_RULE_BAND: {
      int32_t qi = q / r->tile, kj = k / r->tile;
      if (abs(qi - kj) <= r->band) return 1;
      for (int32_t i = 0; i < r->n_global_cols; i++)
        if (r->global_cols[i] == kj) return 1;
      return 0;
    }
    case ORC_RULE_LOCAL: {
      if (q < r->prefix_len || k < r->prefix_len) return 1;
      int32_t fq, yq, xq, fk, yk, xk;
      if (!locate(r, q, &fq, &yq, &xq) || !locate(r, k, &fk, &yk, &xk)) return 0;
      if (abs(fq - fk) <= r->frame_window && abs(yq / r->sp_tile_h - yk / r->sp_tile_h) <= r->sp_window &&
          abs(xq / r->sp_tile_w - xk / r->sp_tile_w) <= r->sp_window)
        return 1;
      return is_landmark(r, fk);
    }
    case ORC_RULE_AXIAL: {
      if (q < r->prefix_len) return 1; /* prefix queries see everything (:129-130) */
      if (k < r->prefix_len) return 1; /* every query keeps the prefix (:131-132) */
      int32_t fq, yq, xq, fk, yk, xk;
      if (!locate(r, q, &fq, &yq, &xq) || !locate(r, k, &fk, &yk, &xk)) return 0;
      if (fq == fk) return 1;             /* same frame */
      if (yq == yk && xq == xk) return 1; /* same position */
      return is_landmark(r, fk);          /* landmark frame */
    }
    default:
      return 0;
  }
}

/* AxialTopology.init(geometry:landmarks:) landmark placement
 * (AxialTopology.swift:82-112): n clamped to [2, f], evenly spaced with both
 * ends, Swift `.rounded()` (ties away from zero == C round()), deduplicated
 * and sorted. */
int orc_landmarks(int32_t frames, int32_t n, int32_t* out) {
  int32_t m = n < frames ? n : frames;
  if (m < 2) m = 2;
  if (m >= frames) {
    for (int32_t i = 0; i < frames; i++) out[i] = i;
    return frames;
  }
  int32_t cnt = 0;
  for (int32_t i = 0; i < m; i++) {
    int32_t v = (int32_t)round((double)i * (double)(frames - 1) / (double)(m - 1));
    int dup = 0;
    for (int32_t j = 0; j < cnt; j++)
      if (out[j] == v) dup = 1;
    if (!dup) out[cnt++] = v;
  }
  /* insertion sort: values are already ascending, kept for safety */
  for (int32_t i = 1; i < cnt; i++) {
    int32_t v = out[i], j = i - 1;
    while (j >= 0 && out[j] > v) { out[j + 1] = out[j]; j--; }
    out[j + 1] = v;
  }
  return cnt;
}

/* AxialTopology.density (AxialTopology.swift:145-170): counted by frame. */
double orc_axial_density_closed(const orc_rule* r) {
  double s = r->seq_len, p = r->prefix_len;
  int64_t per = (int64_t)r->height * r->width;
  int64_t video_allowed = 0;
  for (int32_t f0 = 0; f0 < r->frames; f0++) {
    int64_t full = is_landmark(r, f0) ? r->n_landmarks : r->n_landmarks + 1;
    int64_t per_query = per * full + (r->frames - full);
    video_allowed += per * ((int64_t)p + per_query);
  }
  double total = p * s + (double)video_allowed;
  return total / (s * s);
}

double orc_token_density_counted(const orc_rule* r) {
  int64_t cnt = 0;
  int32_t S = r->seq_len;
#pragma omp parallel for reduction(+ : cnt) schedule(dynamic, 16)
  for (int32_t q = 0; q < S; q++)
    for (int32_t k = 0; k < S; k++) cnt += orc_allows(r, q, k);
  return (double)cnt / ((double)S * (double)S);
}

/* ------------------------------------------------------------ tile lists */

/* Brute force: a tile is active iff any valid token pair inside it is
 * allowed. This is the definition the fast GPU builder must reproduce bit for
 * bit (the reference's bulk-vs-pairwise check, AxialReferenceTests.swift:99-117,
 * carried to tiles). */
int orc_tile_bitmap(const orc_rule* r, int32_t nq, int32_t nk, uint8_t* out) {
  const int32_t T = r->tile, S = r->seq_len;
#pragma omp parallel for schedule(dynamic, 1)
  for (int32_t qi = 0; qi < nq; qi++) {
    for (int32_t kj = 0; kj < nk; kj++) {
      int hit = 0;
      int32_t q0 = qi * T, q1 = q0 + T < S ? q0 + T : S;
      int32_t k0 = kj * T, k1 = k0 + T < S ? k0 + T : S;
      for (int32_t q = q0; q < q1 && !hit; q++)
        for (int32_t k = k0; k < k1; k++)
          if (orc_allows(r, q, k)) { hit = 1; break; }
      out[(int64_t)qi * nk + kj] = (uint8_t)hit;
    }
  }
  return 0;
}

/* CSR: row_ptr[nq+1], ascending column indices per row. */
int64_t orc_csr_from_bitmap(const uint8_t* bm, int32_t nq, int32_t nk,
                            int32_t* row_ptr, int32_t* col_idx) {
  int64_t n = 0;
  for (int32_t i = 0; i < nq; i++) {
    if (row_ptr) row_ptr[i] = (int32_t)n;
    for (int32_t j = 0; j < nk; j++)
      if (bm[(int64_t)i * nk + j]) {
        if (col_idx) col_idx[n] = j;
        n++;
      }
  }
  if (row_ptr) row_ptr[nq] = (int32_t)n;
  return n;
}

/* ------------------------------------------------------------- attention */

static inline int tile_on(const uint8_t* bm, int32_t tile, int32_t nk, int32_t q, int32_t k) {
  return bm[(int64_t)(q / tile) * nk + (k / tile)];
}

/* One query row of AxialReference.attend (AxialReference.swift:89-114): scores
 * over all S keys, additive mask of 0 / -1e30 (maskRows, :78-82), softmax over
 * the union, weighted sum of V. A row with no allowed key returns 0, the
 * l == 0 guard of the streaming form (:163-167); the reference's own fp32
 * sentinel arithmetic would give mean(V) there, and its topology never
 * produces such a row. */
static void masked_row(const float* qrow, const float* k, const float* v, int32_t S, int32_t D,
                       float scale, const uint8_t* bm, int32_t tile, int32_t nk, int32_t qidx,
                       float* scores, double* acc, float* out) {
  float mx = -3.0e38f;
  int any = 0;
  for (int32_t j = 0; j < S; j++) {
    const float* kr = k + (int64_t)j * D;
    float dot = 0.f;
    for (int32_t d = 0; d < D; d++) dot += qrow[d] * kr[d];
    float s = dot * scale + (tile_on(bm, tile, nk, qidx, j) ? 0.0f : -1.0e30f);
    any |= tile_on(bm, tile, nk, qidx, j);
    scores[j] = s;
    if (s > mx) mx = s;
  }
  for (int32_t d = 0; d < D; d++) acc[d] = 0.0;
  if (!any) {
    for (int32_t d = 0; d < D; d++) out[d] = 0.f;
    return;
  }
  double l = 0.0;
  for (int32_t j = 0; j < S; j++) {
    float p = expf(scores[j] - mx);
    if (p == 0.f) continue;
    l += p;
    const float* vr = v + (int64_t)j * D;
    for (int32_t d = 0; d < D; d++) acc[d] += (double)p * vr[d];
  }
  for (int32_t d = 0; d < D; d++) out[d] = (float)(acc[d] / l);
}

void orc_attend_masked(const float* q, const float* k, const float* v,
                       int32_t H, int32_t S, int32_t D, float scale,
                       const uint8_t* bm, int32_t tile, int32_t nk,
                       int32_t query_chunk, int32_t q_lo, int32_t q_hi,
                       int32_t n_threads, float* out) {
  if (query_chunk <= 0) query_chunk = 512;
  int32_t n_chunks = (q_hi - q_lo + query_chunk - 1) / query_chunk;
  int64_t units = (int64_t)H * n_chunks;
#ifdef _OPENMP
  if (n_threads > 0) omp_set_num_threads(n_threads);
#endif
#pragma omp parallel
  {
    float* scores = (float*)malloc(sizeof(float) * (size_t)S);
    double* acc = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(dynamic, 1)
    for (int64_t u = 0; u < units; u++) {
      int32_t h = (int32_t)(u / n_chunks), c = (int32_t)(u % n_chunks);
      int32_t lo = q_lo + c * query_chunk;
      int32_t hi = lo + query_chunk < q_hi ? lo + query_chunk : q_hi;
      const float* kh = k + (int64_t)h * S * D;
      const float* vh = v + (int64_t)h * S * D;
      for (int32_t i = lo; i < hi; i++)
        masked_row(q + ((int64_t)h * S + i) * D, kh, vh, S, D, scale, bm, tile, nk, i, scores, acc,
                   out + ((int64_t)h * S + i) * D);
    }
    free(scores);
    free(acc);
  }
}

void orc_attend_masked_rows(const float* q_rows, int32_t n_rows, const int32_t* rows,
                            const float* k, const float* v, int32_t S, int32_t D, float scale,
                            const uint8_t* bm, int32_t tile, int32_t nk, int32_t n_threads,
                            float* out) {
#ifdef _OPENMP
  if (n_threads > 0) omp_set_num_threads(n_threads);
#endif
#pragma omp parallel
  {
    float* scores = (float*)malloc(sizeof(float) * (size_t)S);
    double* acc = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(dynamic, 4)
    for (int32_t i = 0; i < n_rows; i++)
      masked_row(q_rows + (int64_t)i * D, k, v, S, D, scale, bm, tile, nk, rows[i], scores, acc,
                 out + (int64_t)i * D);
    free(scores);
    free(acc);
  }
}

/* AxialReference.attendStreamingKeys (AxialReference.swift:129-171), in fp32
 * exactly as written: m starts at -3e38 (:142), masked scores carry the
 * -1e30 sentinel, l and acc are rescaled by exp(m - m_new) per key tile
 * (:151-160), and the output is acc / max(l, 1e-30) (:167). */
void orc_attend_streaming(const float* q, const float* k, const float* v,
                          int32_t H, int32_t S, int32_t D, float scale,
                          const uint8_t* bm, int32_t tile, int32_t nk,
                          int32_t query_chunk, int32_t key_tile,
                          int32_t n_threads, float* out) {
  if (query_chunk <= 0) query_chunk = 512;
  if (key_tile <= 0) key_tile = 1024;
  int32_t n_chunks = (S + query_chunk - 1) / query_chunk;
  int64_t units = (int64_t)H * n_chunks;
#ifdef _OPENMP
  if (n_threads > 0) omp_set_num_threads(n_threads);
#endif
#pragma omp parallel
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)key_tile);
    float* acc = (float*)malloc(sizeof(float) * (size_t)D);
#pragma omp for schedule(dynamic, 1)
    for (int64_t u = 0; u < units; u++) {
      int32_t h = (int32_t)(u / n_chunks), c = (int32_t)(u % n_chunks);
      int32_t lo = c * query_chunk, hi = lo + query_chunk < S ? lo + query_chunk : S;
      const float* kh = k + (int64_t)h * S * D;
      const float* vh = v + (int64_t)h * S * D;
      for (int32_t i = lo; i < hi; i++) {
        const float* qr = q + ((int64_t)h * S + i) * D;
        float m = -3.0e38f, l = 0.f;
        for (int32_t d = 0; d < D; d++) acc[d] = 0.f;
        for (int32_t k_lo = 0; k_lo < S; k_lo += key_tile) {
          int32_t k_hi = k_lo + key_tile < S ? k_lo + key_tile : S;
          float tmax = -3.0e38f;
          for (int32_t j = k_lo; j < k_hi; j++) {
            const float* kr = kh + (int64_t)j * D;
            float dot = 0.f;
            for (int32_t d = 0; d < D; d++) dot += qr[d] * kr[d];
            float s = dot * scale + (tile_on(bm, tile, nk, i, j) ? 0.0f : -1.0e30f);
            sc[j - k_lo] = s;
            if (s > tmax) tmax = s;
          }
          float m_new = m > tmax ? m : tmax;
          float rescale = expf(m - m_new);
          float psum = 0.f;
          for (int32_t d = 0; d < D; d++) acc[d] *= rescale;
          for (int32_t j = k_lo; j < k_hi; j++) {
            float p = expf(sc[j - k_lo] - m_new);
            psum += p;
            const float* vr = vh + (int64_t)j * D;
            for (int32_t d = 0; d < D; d++) acc[d] += p * vr[d];
          }
          l = l * rescale + psum;
          m = m_new;
        }
        float den = l > 1e-30f ? l : 1e-30f;
        float* o = out + ((int64_t)h * S + i) * D;
        for (int32_t d = 0; d < D; d++) o[d] = acc[d] / den;
      }
    }
    free(sc);
    free(acc);
  }
}

/* -------------------------------------------------------------- prologue */

/* H3RMSNorm then SplitHalfRoPE, per (token, head) row:
 *   H3RMSNorm (Sources/H3Modules/Modulation.swift:116-120):
 *     f = fp32(x); n = f * rsqrt(mean(f*f) + eps); y = bf16(n * fp32(gamma)),
 *     the mean in the fixed order of mean_square_fixed_order (D == 128),
 *     rsqrt in double rounded once to fp32
 *   RoPE angle (Sources/H3Modules/H3Transformer.swift:66-78):
 *     angle = fp32(pos[axis]) * inv_freq (fp32); table = bf16([[c,-s],[s,c]]),
 *     c and s the fp32-rounded cos/sin of the fp32 angle
 *   SplitHalfRoPE (Sources/H3Modules/DiTBlock.swift:83-103), with the bf16
 *   rounding of every product and sum that MLX applies on bf16 arrays and the
 *   fused fixture mirrors (Tests/H3ModulesTests/QKFusionMetalFixture.swift:57-69):
 *     ra = bf16(bf16(c*a) + bf16(-s*b)); rb = bf16(bf16(s*a) + bf16(c*b))
 *   pairs (p, p + rot/2), channels >= rot pass through.
 * ORC_ROUND_FP32 keeps the normalised row and the rotation in fp32 and rounds
 * once at the store. Output is head-major [H, S_pad, D]; rows >= S are zero. */
/* The mean of squares over a 128-channel row in the fixed fp32 order the
 * prologue defines (the reference's MLX reduction order is not observable):
 * the row is split into 8 pieces of two 8-channel chunks -- piece j holds
 * chunks j and j + rot/16 while 8j < rot/2, else two consecutive chunks of the
 * channels >= rot -- each piece is summed with fma in channel order, and the 8
 * piece sums combine as t_j = s_j + s_{7-j}, u_j = t_j + t_{j^2}, u_0 + u_1. */
static float mean_square_fixed_order(const float* f, int32_t rot) {
  const int32_t hl = rot / 16;
  float sj[8];
  for (int32_t j = 0; j < 8; j++) {
    int32_t ca = j < hl ? j : 2 * hl + 2 * (j - hl);
    int32_t cb = j < hl ? j + hl : ca + 1;
    float acc = 0.f;
    for (int32_t i = 0; i < 8; i++) acc = fmaf(f[8 * ca + i], f[8 * ca + i], acc);
    for (int32_t i = 0; i < 8; i++) acc = fmaf(f[8 * cb + i], f[8 * cb + i], acc);
    sj[j] = acc;
  }
  float t0 = sj[0] + sj[7], t1 = sj[1] + sj[6], t2 = sj[2] + sj[5], t3 = sj[3] + sj[4];
  float u0 = t0 + t2, u1 = t1 + t3;
  return (u0 + u1) * (1.0f / 128.0f);
}

void orc_qk_norm_rope(const uint16_t* x, int64_t ld, int32_t S, int32_t S_pad,
                      int32_t H, int32_t D, const uint16_t* gamma, float eps,
                      const float* pos, const int32_t* pair_axis, const float* pair_inv,
                      int32_t rot, int32_t mode, int32_t n_threads, uint16_t* out) {
  const int32_t half = rot / 2;
#ifdef _OPENMP
  if (n_threads > 0) omp_set_num_threads(n_threads);
#endif
#pragma omp parallel
  {
    float* f = (float*)malloc(sizeof(float) * (size_t)D);
    float* y = (float*)malloc(sizeof(float) * (size_t)D);
#pragma omp for schedule(static)
    for (int64_t row = 0; row < (int64_t)S_pad * H; row++) {
      int32_t s = (int32_t)(row / H), h = (int32_t)(row % H);
      uint16_t* o = out + ((int64_t)h * S_pad + s) * D;
      if (s >= S) {
        memset(o, 0, sizeof(uint16_t) * (size_t)D);
        continue;
      }
      const uint16_t* xr = x + (int64_t)s * ld + (int64_t)h * D;
      for (int32_t d = 0; d < D; d++) f[d] = orc_bf16_to_f32(xr[d]);
      float ms = mean_square_fixed_order(f, rot);
      float r = (float)(1.0 / sqrt((double)(ms + eps)));
      for (int32_t d = 0; d < D; d++) y[d] = (f[d] * r) * orc_bf16_to_f32(gamma[d]);
      for (int32_t d = 0; d < D; d++) o[d] = orc_f32_to_bf16(y[d]);
      for (int32_t p = 0; p < half; p++) {
        float ang = pos[(int64_t)s * 3 + pair_axis[p]] * pair_inv[p];
        /* cos/sin of the fp32 angle, evaluated in double and rounded once */
        float cf = (float)cos((double)ang), sf = (float)sin((double)ang);
        if (mode == ORC_ROUND_REFERENCE) {
          float c = rbf(cf), sn = rbf(sf), ns = rbf(-sf);
          float a = orc_bf16_to_f32(o[p]), b = orc_bf16_to_f32(o[p + half]);
          o[p] = orc_f32_to_bf16(rbf(c * a) + rbf(ns * b));
          o[p + half] = orc_f32_to_bf16(rbf(sn * a) + rbf(c * b));
        } else {
          float a = y[p], b = y[p + half];
          o[p] = orc_f32_to_bf16(cf * a + (-sf) * b);
          o[p + half] = orc_f32_to_bf16(sf * a + cf * b);
        }
      }
    }
    free(f);
    free(y);
  }
}

/* H3RoPE.rotationTable(angles(pos, inv_freq)) in the compute dtype
 * (Sources/H3Modules/H3Transformer.swift:62-78, built once per render at
 * :271-273): per token s and pair p the 2x2 block [[c, -s], [s, c]] stored
 * row-major as (c, -s, s, c), with angle = fp32(pos[s][axis[p]]) * inv[p] and
 * c, s its cos/sin evaluated in double and rounded once to fp32 -- the values
 * orc_qk_norm_rope rotates with. ORC_ROUND_REFERENCE: bf16 entries (uint16
 * bit patterns, the bf16 table the reference casts to); ORC_ROUND_FP32: fp32
 * entries. out holds S * half * 4 entries. */
void orc_rope_table(const float* pos, int32_t S, const int32_t* pair_axis,
                    const float* pair_inv, int32_t half, int32_t mode, void* out) {
  for (int64_t s = 0; s < S; s++) {
    for (int32_t p = 0; p < half; p++) {
      float ang = pos[s * 3 + pair_axis[p]] * pair_inv[p];
      float cf = (float)cos((double)ang), sf = (float)sin((double)ang);
      int64_t e = (s * half + p) * 4;
      if (mode == ORC_ROUND_REFERENCE) {
        uint16_t* o = (uint16_t*)out;
        o[e] = orc_f32_to_bf16(cf);
        o[e + 1] = orc_f32_to_bf16(-sf);
        o[e + 2] = orc_f32_to_bf16(sf);
        o[e + 3] = orc_f32_to_bf16(cf);
      } else {
        float* o = (float*)out;
        o[e] = cf;
        o[e + 1] = -sf;
        o[e + 2] = sf;
        o[e + 3] = cf;
      }
    }
  }
}

/* ------------------------------------------------- RoPE tables, positions */

/* Three-axis RoPE for the synthetic benchmark shapes: dim_t/dim_h/dim_w
 * channels per axis (pairs = dim/2 each, in t|h|w order), inv_freq[i] =
 * theta^(-2i/dim_axis) computed in double and narrowed to fp32. */
int orc_rope_pairs_axes(double theta, int32_t dim_t, int32_t dim_h, int32_t dim_w,
                        int32_t* pair_axis, float* pair_inv) {
  int32_t dims[3] = {dim_t, dim_h, dim_w};
  int32_t p = 0;
  for (int32_t a = 0; a < 3; a++)
    for (int32_t i = 0; i < dims[a] / 2; i++) {
      pair_axis[p] = a;
      pair_inv[p] = (float)(1.0 / pow(theta, 2.0 * (double)i / (double)dims[a]));
      p++;
    }
  return p;
}

/* H3RoPE.angles (H3Transformer.swift:64-70): every axis uses the same n_freq
 * checkpoint frequencies and the pairs are ordered t|h|w, so pair p rotates by
 * pos[p / n_freq] * inv_freq[p % n_freq] and rot = 6 * n_freq channels. */
int orc_rope_pairs_h3(const float* inv_freq, int32_t n_freq, int32_t* pair_axis, float* pair_inv) {
  for (int32_t p = 0; p < 3 * n_freq; p++) {
    pair_axis[p] = p / n_freq;
    pair_inv[p] = inv_freq[p % n_freq];
  }
  return 3 * n_freq;
}

/* Synthetic benchmark positions: prefix tokens at (0,0,0), video token
 * (t, y, x) at its integer lattice coordinates. */
void orc_positions_grid(int32_t prefix_len, int32_t frames, int32_t height, int32_t width,
                        float* pos) {
  int64_t i = 0;
  for (int32_t p = 0; p < prefix_len; p++, i++) pos[i * 3] = pos[i * 3 + 1] = pos[i * 3 + 2] = 0.f;
  for (int32_t t = 0; t < frames; t++)
    for (int32_t y = 0; y < height; y++)
      for (int32_t x = 0; x < width; x++, i++) {
        pos[i * 3] = (float)t;
        pos[i * 3 + 1] = (float)y;
        pos[i * 3 + 2] = (float)x;
      }
}

/* PositionGrid.axis (Sources/H3Foundation/PackedSequence.swift:66-76). */
static int grid_axis(int32_t dim, int32_t patch, double sqrt_area, double* out) {
  double ratio = (double)dim / sqrt_area;
  int32_t n = dim / patch;
  if (n <= 0) return -1;
  double step = ratio / (double)n, origin = (1.0 - ratio) / 2.0;
  for (int32_t i = 0; i < n; i++) out[i] = ((double)i * step + origin) * 32.0;
  return n;
}

/* PackedLayout.positionIds for text | target audio | target video
 * (PackedSequence.swift:185-296, no keyframes or references): text i at
 * (i,0,0); audio at (text + i, 0, w_lo) then (text + i, 0, w_hi); video frames
 * on videoTGrid (5/3 * [1,4,4,4,4] spans, :94-103) times the area-normalised
 * (h, w) grid (:80-91). Double precision, as the reference builds it. */
int orc_positions_packed(int32_t text_tokens, int32_t audio_t, int32_t latent_t,
                         int32_t latent_h, int32_t latent_w, int32_t patch, double* pos) {
  double area = sqrt((double)latent_h * (double)latent_w);
  double* ha = (double*)malloc(sizeof(double) * (size_t)(latent_h + 1));
  double* wa = (double*)malloc(sizeof(double) * (size_t)(latent_w + 1));
  int32_t nh = grid_axis(latent_h, patch, area, ha), nw = grid_axis(latent_w, patch, area, wa);
  if (nh <= 0 || nw <= 0) {
    free(ha);
    free(wa);
    return -1;
  }
  int64_t i = 0;
  for (int32_t t = 0; t < text_tokens; t++, i++) {
    pos[i * 3] = (double)t;
    pos[i * 3 + 1] = 0.0;
    pos[i * 3 + 2] = 0.0;
  }
  double cursor = (double)text_tokens;
  double wl = wa[0], wh = wa[nw - 1];
  for (int side = 0; side < 2; side++)
    for (int32_t a = 0; a < audio_t; a++, i++) {
      pos[i * 3] = cursor + (double)a;
      pos[i * 3 + 1] = 0.0;
      pos[i * 3 + 2] = side ? wh : wl;
    }
  static const int fpt[5] = {1, 4, 4, 4, 4};
  double acc = cursor;
  for (int32_t t = 0; t < latent_t; t++) {
    for (int32_t y = 0; y < nh; y++)
      for (int32_t x = 0; x < nw; x++, i++) {
        pos[i * 3] = acc;
        pos[i * 3 + 1] = ha[y];
        pos[i * 3 + 2] = wa[x];
      }
    acc += (5.0 / 3.0) * (double)fpt[t % 5];
  }
  free(ha);
  free(wa);
  return (int)i;
}
