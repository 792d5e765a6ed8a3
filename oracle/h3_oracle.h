/*
 * h3_oracle.h -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * CPU restatement of the reference's DiT attention hot path, used only as the
 * checker: by tests/, by __graft_entry__.smoke() and by bench.py's
 * cpu_baseline leg. Nothing in the shipped library links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the loading-awesome/MiniMax-H3-Swift tree). Where the reference leaves a
 * choice open (tile-level mask rules for the synthetic benchmark shapes), the
 * rule is written down here and the product implements the same written rule.
 */
#ifndef H3_ORACLE_H
#define H3_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ORC_RULE_DENSE = 0,   /* every (q,k) with q,k < S */
  ORC_RULE_BAND = 1,    /* tile level: |qi-kj| <= band, or kj a global column */
  ORC_RULE_LOCAL = 2,   /* token level: prefix rows/cols + +-frame window + spatial-tile window (+ landmark frames) */
  ORC_RULE_AXIAL = 3,   /* token level: AxialTopology.allows (prefix, same frame, same (y,x), landmark frames) */
};

typedef struct {
  int32_t kind;
  int32_t seq_len;        /* S: valid tokens */
  int32_t tile;           /* tile edge in tokens (128 on the product path) */
  int32_t prefix_len;     /* rows before the video span: text | cond | audio */
  int32_t frames, height, width;  /* video lattice; frames*height*width == seq_len - prefix_len */
  int32_t frame_window;   /* LOCAL: |t_q - t_k| <= frame_window */
  int32_t sp_tile_h, sp_tile_w;   /* LOCAL: spatial tile edge in latent tokens */
  int32_t sp_window;      /* LOCAL: |tile_q - tile_k| <= sp_window per spatial axis */
  int32_t band;           /* BAND: diagonal half-width in tiles */
  int32_t n_global_cols;  /* BAND: tile columns every row sees */
  const int32_t* global_cols;
  int32_t n_landmarks;    /* LOCAL/AXIAL: frames every video query sees in full */
  const int32_t* landmarks;
} orc_rule;

/* bf16 <-> fp32, round to nearest even (NaN kept quiet). */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n);
void orc_bf16_to_f32_n(const uint16_t* in, float* out, int64_t n);

/* ---- topology (AxialTopology.swift) ---- */
int orc_allows(const orc_rule* r, int32_t q, int32_t k);
int orc_landmarks(int32_t frames, int32_t n, int32_t* out);        /* returns count */
double orc_axial_density_closed(const orc_rule* r);                /* AxialTopology.density */
double orc_token_density_counted(const orc_rule* r);               /* counted over S^2 pairs */

/* ---- tile lists (brute force; OR over token pairs) ---- */
int orc_tile_bitmap(const orc_rule* r, int32_t nq, int32_t nk, uint8_t* out);
int64_t orc_csr_from_bitmap(const uint8_t* bm, int32_t nq, int32_t nk,
                            int32_t* row_ptr, int32_t* col_idx);

/* ---- attention (AxialReference.swift) ---- */
/* q,k,v: fp32 [H, S, D] contiguous. bm: tile bitmap [nq, nk] at `tile`.
 * Rows [q_lo, q_hi) of every head are written into out [H, S, D]. */
void orc_attend_masked(const float* q, const float* k, const float* v,
                       int32_t H, int32_t S, int32_t D, float scale,
                       const uint8_t* bm, int32_t tile, int32_t nk,
                       int32_t query_chunk, int32_t q_lo, int32_t q_hi,
                       int32_t n_threads, float* out);
void orc_attend_streaming(const float* q, const float* k, const float* v,
                          int32_t H, int32_t S, int32_t D, float scale,
                          const uint8_t* bm, int32_t tile, int32_t nk,
                          int32_t query_chunk, int32_t key_tile,
                          int32_t n_threads, float* out);
/* Rows of one head only, for sampled full-size checks: rows[] lists query rows. */
void orc_attend_masked_rows(const float* q_rows, int32_t n_rows, const int32_t* rows,
                            const float* k, const float* v, int32_t S, int32_t D, float scale,
                            const uint8_t* bm, int32_t tile, int32_t nk, int32_t n_threads,
                            float* out);

/* ---- prologue (Modulation.swift H3RMSNorm, DiTBlock.swift SplitHalfRoPE) ---- */
enum { ORC_ROUND_REFERENCE = 0, ORC_ROUND_FP32 = 1 };
void orc_qk_norm_rope(const uint16_t* x, int64_t ld, int32_t S, int32_t S_pad,
                      int32_t H, int32_t D, const uint16_t* gamma, float eps,
                      const float* pos, const int32_t* pair_axis, const float* pair_inv,
                      int32_t rot, int32_t mode, int32_t n_threads, uint16_t* out);
/* H3RoPE.rotationTable in the compute dtype: (c, -s, s, c) per token and pair,
 * bf16 bit patterns (REFERENCE) or fp32 (FP32), S * half * 4 entries. */
void orc_rope_table(const float* pos, int32_t S, const int32_t* pair_axis,
                    const float* pair_inv, int32_t half, int32_t mode, void* out);

/* ---- RoPE tables and positions (H3Transformer.swift, PackedSequence.swift) ---- */
int orc_rope_pairs_axes(double theta, int32_t dim_t, int32_t dim_h, int32_t dim_w,
                        int32_t* pair_axis, float* pair_inv);
int orc_rope_pairs_h3(const float* inv_freq, int32_t n_freq, int32_t* pair_axis, float* pair_inv);
void orc_positions_grid(int32_t prefix_len, int32_t frames, int32_t height, int32_t width,
                        float* pos);
int orc_positions_packed(int32_t text_tokens, int32_t audio_t, int32_t latent_t,
                         int32_t latent_h, int32_t latent_w, int32_t patch, double* pos);

#ifdef __cplusplus
}
#endif
#endif
