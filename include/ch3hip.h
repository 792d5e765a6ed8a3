/*
 * ch3hip.h -- C ABI of the MI355X (gfx950) DiT attention hot path.
 *
 * Three stages, one process, one GPU:
 *   1. block mask -> active-tile index lists (CSR over 128x128 tiles), held in
 *      an opaque plan built once per shape;
 *   2. fused Q/K RMSNorm + 3D split-half RoPE + relayout to head-major;
 *   3. block-sparse flash attention over the plan's active tiles.
 *
 * Conventions
 *   - Tensors are caller-owned device pointers (bf16 as raw 16-bit words)
 *     with explicit shapes; `stream` is a hipStream_t passed as void* (NULL =
 *     the default stream). Calls are stream-ordered and asynchronous unless a
 *     comment says otherwise; the caller synchronises.
 *   - Return codes: H3HIP_OK (0); H3HIP_DECLINED (1) for a geometry or policy
 *     this path does not take, in which case the caller runs its dense
 *     attention -- the `nil` of H3AttentionBackend.attend
 *     (Sources/H3Attention/AttentionBackend.swift:123-127) and of
 *     FusedQKRoPE.apply (Tests/H3ModulesTests/QKFusionMetalFixture.swift:85-95);
 *     negative values for invalid arguments or HIP failures, never a trap
 *     (the refusal style of Sources/H3Foundation/H3Error.swift).
 *     h3hip_last_error() returns the calling thread's last message.
 *   - Head-major layout is [heads, seq_pad, head_dim], seq_pad = ceil(S/128)*128.
 *     Token-major layout is [S, heads*head_dim] with a row stride.
 */
#ifndef CH3HIP_H
#define CH3HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define H3HIP_OK 0
#define H3HIP_DECLINED 1
#define H3HIP_EINVAL (-1)
#define H3HIP_EHIP (-2)
#define H3HIP_ENOMEM (-3)
#define H3HIP_EDEVICE (-4)

#define H3HIP_TILE 128

/* Mask rule kinds for h3hip_mask_rule.kind. */
#define H3HIP_RULE_DENSE 0  /* every tile: the no-skip "faithful" path */
#define H3HIP_RULE_BAND 1   /* tile level: |qi - kj| <= band, or kj in global_cols */
#define H3HIP_RULE_LOCAL 2  /* token level: prefix rows/cols dense; video pairs within
                               +-frame_window frames and +-spatial_window spatial tiles
                               of spatial_tile_h x spatial_tile_w tokens; + landmark frames */
#define H3HIP_RULE_AXIAL 3  /* token level: the reference's AxialTopology.allows --
                               prefix rows/cols, same frame, same (y,x), landmark frames
                               (Sources/H3Attention/AxialTopology.swift:128-137) */
#define H3HIP_RULE_BITMAP 4 /* caller-supplied tile bitmap */

/* Rounding modes of the prologue. */
#define H3HIP_ROUND_REFERENCE 0 /* bf16 after RMSNorm and after every RoPE product and sum,
                                   as MLX does on bf16 arrays (DiTBlock.swift:83-103) */
#define H3HIP_ROUND_FP32 1      /* fp32 until the single store */

/* Output layouts of the attention. */
#define H3HIP_OUT_HEAD_MAJOR 0  /* [heads, seq_pad, head_dim] */
#define H3HIP_OUT_TOKEN_MAJOR 1 /* [seq_pad, heads*head_dim]: what AttentionLayer.sdpa
                                   hands the out-projection (DiTBlock.swift:323-327) */

/* Which (query, key) pairs may attend. Token-level kinds are OR-reduced onto
 * the 128x128 tile grid: a tile is active iff any valid pair inside it is
 * allowed. Token order is [text | cond/refs | audio | video]
 * (Sources/H3Foundation/PackedSequence.swift:173-176): everything before the
 * video span is the prefix. Replaces AxialTopology's initialisers
 * (AxialTopology.swift:65-112); unused fields are ignored by a kind. */
typedef struct {
  int32_t kind;
  int32_t seq_len;        /* S: valid tokens (padding to seq_pad is never attended) */
  int32_t prefix_len;     /* tokens before the video span */
  int32_t frames;         /* video lattice; frames*height*width == seq_len - prefix_len */
  int32_t height;
  int32_t width;
  int32_t frame_window;   /* LOCAL */
  int32_t spatial_tile_h; /* LOCAL */
  int32_t spatial_tile_w; /* LOCAL */
  int32_t spatial_window; /* LOCAL */
  int32_t band;           /* BAND */
  int32_t n_global_cols;  /* BAND */
  const int32_t* global_cols;
  int32_t n_landmarks;    /* LOCAL, AXIAL: host array of frame indices */
  const int32_t* landmark_frames;
  const uint8_t* bitmap;  /* BITMAP: host [n_tiles * n_tiles] row-major, nonzero = active */
} h3hip_mask_rule;

/* When the backend declines a call so the caller runs dense: the policy a
 * sparse backend expresses through AttentionContext
 * (Sources/H3Attention/AttentionBackend.swift:10-59). Zero-initialised = never. */
typedef struct {
  int32_t dense_first_blocks;   /* blocks [0, n) stay dense */
  int32_t dense_last_blocks;    /* blocks [count - n, count) stay dense */
  double dense_until_progress;  /* schedule progress below this stays dense (warm-up) */
  int32_t min_sequence_length;  /* shorter sequences stay dense */
} h3hip_policy;

/* AttentionContext (AttentionBackend.swift:37-59). video_start < 0 means nil. */
typedef struct {
  int32_t block_index;
  int32_t block_count;
  double schedule_progress;
  int32_t sequence_length;
  int32_t video_start;
  int32_t video_stop;
} h3hip_attention_context;

typedef struct h3hip_plan_s* h3hip_plan;

/* ---------------------------------------------------------------- device */

/* H3AttentionBackend.isAvailable(on:) (AttentionBackend.swift:93-94): 1 if
 * `device` is a gfx950 GPU this library's kernels were built for, else 0. */
int h3hip_device_supported(int32_t device);
const char* h3hip_last_error(void);
const char* h3hip_version(void);

/* ----------------------------------------------------------------- plans */

/* Builds the tile lists on the current device (synchronous). Replaces the
 * topology construction of AxialTopology.init (AxialTopology.swift:65-112) and
 * the Sol-Attn routing stage (docs/SOL_ATTN.md:42-72): a plan is built once
 * per shape ("precomputable once per render", AxialTopology.swift:17-18) and
 * reused by every block. `heads` fixes the launch schedule; `policy` may be NULL. */
int h3hip_plan_create(const h3hip_mask_rule* rule, int32_t heads, const h3hip_policy* policy,
                      void* stream, h3hip_plan* out);
int h3hip_plan_destroy(h3hip_plan plan);
/* Shape and list size. Any output pointer may be NULL. */
int h3hip_plan_info(h3hip_plan plan, int32_t* seq_len, int32_t* seq_pad, int32_t* n_tiles,
                    int64_t* nnz, int32_t* heads);
/* Copies the CSR lists (host): row_ptr[n_tiles + 1], col_idx[nnz], columns
 * ascending per row. Bit-exact export for tests and callers. */
int h3hip_plan_tiles(h3hip_plan plan, int32_t* row_ptr, int32_t* col_idx);
/* Counted tile density nnz / n_tiles^2 -- AxialTopology.density's role
 * (AxialTopology.swift:139-170), counted on tiles. */
double h3hip_plan_density(h3hip_plan plan);

/* The attention launch's persistent schedule for a plan with these CSR rows
 * (host-side, synchronous; h3hip_plan_create builds the same lists). No
 * counterpart in the reference, whose MLX dispatch has no persistent
 * workgroups; exposed so callers and tests can inspect which (head, q-tile)
 * units each workgroup runs. row_ptr[n_tiles + 1]; groups = workgroups, a
 * positive multiple of 8 (one per CU: 256 on MI355X). Writes
 * work_ptr[groups + 1] and work[heads * n_tiles]: workgroup b runs units
 * work[work_ptr[b] .. work_ptr[b + 1]) in order, each (head << 16 | q_tile),
 * every unit exactly once. */
int h3hip_schedule(const int32_t* row_ptr, int32_t n_tiles, int32_t heads, int32_t groups,
                   int32_t* work_ptr, int32_t* work);

/* ------------------------------------------------------- tile-list builder */

/* Device tile bitmap from a token-level rule: d_bitmap [n_tiles * n_tiles]
 * bytes, 1 = active. Asynchronous. AxialReference.maskRows's role
 * (Sources/H3Attention/AxialReference.swift:42-84), reduced onto tiles. */
int h3hip_mask_from_rule(const h3hip_mask_rule* rule, uint8_t* d_bitmap, void* stream);

/* h3hip_mask_from_rule without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The rule's flag tables (BAND global columns, landmark frames) are built in a
 * static per-GPU scratch array of 192 KiB inside the library instead of a
 * temporary allocation: at most 32,768 flags (tile columns or frames) and
 * 32,768 listed entries; larger rules are refused with H3HIP_EINVAL. Same
 * bitmap as h3hip_mask_from_rule.
 * Lists of up to 256 entries (global columns or landmark frames) travel by
 * value in the kernel arguments: nothing is copied from host memory and
 * nothing synchronises, so DENSE, BAND, LOCAL and AXIAL rules with such lists
 * can be captured into a HIP graph and replayed (the host lists may be freed
 * after the call). Longer lists are staged from host memory and `stream` is
 * synchronised before returning; BITMAP rules copy the host bitmap and
 * synchronise. Under stream capture both of those are refused with
 * H3HIP_EINVAL and capture is left intact.
 * Every call on one GPU shares that GPU's scratch: calls that overlap on one
 * GPU (concurrent streams or threads, or replays of graphs holding this call)
 * race. */
int h3hip_mask_from_rule_noalloc(const h3hip_mask_rule* rule, uint8_t* d_bitmap, void* stream);

/* Block mask -> CSR on the device. d_bitmap [nq * nk] bytes; d_row_ptr[nq + 1]
 * and d_col_idx[col_capacity] are written. Synchronises `stream` once to read
 * nnz; returns H3HIP_EINVAL (with *nnz set) if col_capacity < nnz. Ascending
 * columns per row. */
int h3hip_tiles_from_mask(const uint8_t* d_bitmap, int32_t nq, int32_t nk, int32_t* d_row_ptr,
                          int32_t* d_col_idx, int64_t col_capacity, int64_t* nnz, void* stream);

/* --------------------------------------------------------------- prologue */

/* Fused H3RMSNorm (Sources/H3Modules/Modulation.swift:116-120) -> split-half
 * RoPE (DiTBlock.swift:83-103, table from H3Transformer.swift:72-78) ->
 * head-major relayout, in one pass over Q and K. Replaces the inline
 * qNorm/kNorm/RoPE of AttentionLayer.callAsFunction (DiTBlock.swift:346-352)
 * and FusedQKRoPE.apply (QKFusionMetalFixture.swift:82-108).
 *   q_in, k_in: device bf16, token-major, row stride ld_in elements
 *               (q_in = qkv, k_in = qkv + heads*head_dim, ld_in = 3*heads*head_dim
 *               for the fused blocked Q|K|V projection).
 *   v_in:       optional (NULL = skip); copied to v_out head-major, unchanged.
 *   q_gamma, k_gamma: device bf16 [head_dim].
 *   pos:        device fp32 [seq_len, 3] (t, h, w).
 *   pair_axis, pair_inv_freq: device [rot/2]; pair p rotates channels (p, p + rot/2)
 *               by pos[axis] * inv_freq; channels >= rot pass through.
 *   q_out, k_out, v_out: device bf16 [heads, seq_pad, head_dim]; rows >= seq_len are zeroed.
 * Declines (returns H3HIP_DECLINED) unless head_dim == 128, rot % 16 == 0 and
 * rot <= head_dim, as the fixture declines unsupported geometry. */
int h3hip_qk_norm_rope(const void* q_in, const void* k_in, int64_t ld_in, const void* v_in,
                       const void* q_gamma, const void* k_gamma, float eps, const float* pos,
                       const int32_t* pair_axis, const float* pair_inv_freq, int32_t rot,
                       int32_t rounding, int32_t seq_len, int32_t seq_pad, int32_t heads,
                       int32_t head_dim, void* q_out, void* k_out, void* v_out, void* stream);

/* Token-major -> head-major copy: the [S, heads, head_dim] -> [heads, S, head_dim]
 * transposes of AttentionLayer.sdpa (Sources/H3Modules/DiTBlock.swift:297-300)
 * materialised. in: device bf16 [seq_len, >= heads*head_dim], row stride ld_in
 * elements (V of a fused Q|K|V projection: in = qkv + 2*heads*head_dim,
 * ld_in = 3*heads*head_dim). out: device bf16 [heads, seq_pad, head_dim]; rows
 * >= seq_len are zeroed. No arithmetic: every row is moved unchanged.
 * Declines unless head_dim == 128. */
int h3hip_head_major(const void* in, int64_t ld_in, int32_t seq_len, int32_t seq_pad,
                     int32_t heads, int32_t head_dim, void* out, void* stream);

/* The rotation table of a render: H3RoPE.rotationTable(H3RoPE.angles(pos,
 * inv_freq)) (Sources/H3Modules/H3Transformer.swift:62-78), which
 * prepareRender builds once per render (:271-273) and every layer's
 * AttentionLayer.callAsFunction(_:ropeTable:) takes (DiTBlock.swift:336).
 *   pos, pair_axis, pair_inv_freq, rot: as for h3hip_qk_norm_rope.
 *   table: device [seq_len, rot/2, 2, 2] holding [[c, -s], [s, c]] per token and
 *          pair: bf16 for H3HIP_ROUND_REFERENCE (the reference's bf16 table),
 *          fp32 for H3HIP_ROUND_FP32; 16-byte aligned.
 * The entries are the ones h3hip_qk_norm_rope rotates with. */
int h3hip_rope_table(const float* pos, const int32_t* pair_axis, const float* pair_inv_freq,
                     int32_t rot, int32_t rounding, int32_t seq_len, void* table, void* stream);

/* The QKV projection of AttentionLayer.callAsFunction (DiTBlock.swift:336-345:
 * qkv = x . qkvWeight^T, split into Q | K | V) with the Q/K prologue of
 * DiTBlock.swift:346-352 (what h3hip_qk_norm_rope does) fused into the GEMM's
 * epilogue, so the token-major qkv is never written. Q and K come out equal,
 * bit for bit, to h3hip_qk_norm_rope applied to the bf16-rounded projection;
 * V is the bf16 projection, head-major.
 *   x:      device bf16 [seq_len, hidden], row stride ldx elements.
 *   w:      device bf16 [3*heads*head_dim, hidden] (qkvWeight, Q | K | V rows),
 *           row stride ldw elements.
 *   q_gamma, k_gamma, eps, rot, rounding: as for h3hip_qk_norm_rope.
 *   rope_table: the render's rotation table (the ropeTable argument), as
 *           h3hip_rope_table writes it for this rounding mode: bf16 for
 *           REFERENCE -- the reference's own table -- or fp32 for FP32.
 *   With both gammas NULL the call is the plain GEMM: all three parts written
 *   unchanged (head-major), rope_table unused.
 *   q_out, k_out, v_out: device bf16 [heads, seq_pad, head_dim]; rows >= seq_len
 *           are zeroed.
 * Declines unless head_dim == 128, rot is 96 or 128, heads is even and hidden
 * is a multiple of 64. */
int h3hip_qkv_proj(const void* x, int64_t ldx, const void* w, int64_t ldw, int32_t hidden,
                   const void* q_gamma, const void* k_gamma, float eps, const void* rope_table,
                   int32_t rot, int32_t rounding, int32_t seq_len, int32_t seq_pad,
                   int32_t heads, int32_t head_dim, void* q_out, void* k_out, void* v_out,
                   void* stream);

/* The out-projection of AttentionLayer.callAsFunction (DiTBlock.swift:359:
 * matmul(merged, outWeight.T), no bias): y = x . w^T in bf16 with fp32
 * accumulation, on the same MFMA main loop as h3hip_qkv_proj, written
 * token-major.
 *   x: device bf16 [seq_len, in_features] (the attention output, token-major
 *      [S, heads*head_dim]), row stride ldx elements.
 *   w: device bf16 [out_features, in_features] (outWeight), row stride ldw.
 *   y: device bf16 [seq_len, out_features], row stride ldy; rows < seq_len
 *      written.
 * Declines unless in_features is a multiple of 64 and out_features a
 * multiple of 256. */
int h3hip_out_proj(const void* x, int64_t ldx, const void* w, int64_t ldw, int32_t in_features,
                   int32_t out_features, int32_t seq_len, void* y, int64_t ldy, void* stream);

/* -------------------------------------------------------------- attention */

/* Block-sparse attention over the plan's active tiles: for each query row,
 * one softmax over the union of its active key tiles (keys >= seq_len
 * excluded), the recurrence of AxialReference.attendStreamingKeys
 * (AxialReference.swift:129-171) run on 128-key tiles. q, k, v: device bf16
 * [heads, seq_pad, head_dim]. out: bf16 in `out_layout`; rows >= seq_len and
 * rows with no active tile are zero. Replaces the MLXFast SDPA dispatch of
 * SDPABackend.attend (AttentionBackend.swift:141-154). Declines unless
 * head_dim == 128 and heads == the plan's heads. */
int h3hip_bsattn_fwd(h3hip_plan plan, const void* q, const void* k, const void* v, int32_t heads,
                     int32_t head_dim, float scale, void* out, int32_t out_layout, void* stream);

/* A [heads, rows, head_dim] bf16 view of a caller tensor: element (h, s, d)
 * at data + h*head_stride + s*row_stride + d (strides in elements, multiples
 * of 8; row_stride >= head_dim). A head-major buffer is {seq_pad*128, 128};
 * V straight out of a fused token-major Q|K|V projection is
 * {128, 3*heads*128} at qkv + 2*heads*128. */
typedef struct {
  void* data;
  int64_t head_stride;
  int64_t row_stride;
} h3hip_view;

/* h3hip_bsattn_fwd on strided views, the arrays SDPABackend.attend receives
 * (AttentionBackend.swift:141-154): AttentionLayer hands it lazily transposed
 * [B, H, S, D] views of the projection (DiTBlock.swift:323-327, 346-352), so
 * V needs no copy. Reads rows < seq_len of q, k, v only (no padding rows
 * need exist) and writes rows < seq_len of out; rows with no active tile are
 * zero. K and V rows are fetched with 32-bit offsets: seq_pad * row_stride * 2
 * must stay below 2^31. Same declines as h3hip_bsattn_fwd. */
int h3hip_bsattn_fwd_strided(h3hip_plan plan, const h3hip_view* q, const h3hip_view* k,
                             const h3hip_view* v, int32_t heads, int32_t head_dim, float scale,
                             const h3hip_view* out, void* stream);

/* H3AttentionBackend.attend (AttentionBackend.swift:123-127) with its context:
 * applies the plan's policy and geometry checks, then runs h3hip_bsattn_fwd
 * with a head-major output. H3HIP_DECLINED = the caller runs dense. */
int h3hip_attend(h3hip_plan plan, const h3hip_attention_context* ctx, const void* q,
                 const void* k, const void* v, int32_t heads, int32_t head_dim, float scale,
                 void* out, void* stream);

/* H3AttentionBackend.attend (AttentionBackend.swift:123-127) on the strided
 * [B, H, S, D] views the backend receives from AttentionLayer.sdpa
 * (DiTBlock.swift:293-316): the policy and geometry checks of h3hip_attend,
 * then h3hip_bsattn_fwd_strided. No padding or copy is needed on either side;
 * rows < seq_len of out are written. */
int h3hip_attend_strided(h3hip_plan plan, const h3hip_attention_context* ctx,
                         const h3hip_view* q, const h3hip_view* k, const h3hip_view* v,
                         int32_t heads, int32_t head_dim, float scale, const h3hip_view* out,
                         void* stream);

/* ------------------------------------------------- host-side table helpers */

/* Three-axis RoPE pair table: dim_t/dim_h/dim_w channels per axis in t|h|w
 * order, inv_freq[i] = theta^(-2i/dim_axis) (double, narrowed to fp32).
 * Writes (dim_t+dim_h+dim_w)/2 entries; returns the count. */
int h3hip_rope_pairs_axes(double theta, int32_t dim_t, int32_t dim_h, int32_t dim_w,
                          int32_t* pair_axis, float* pair_inv_freq);
/* H3RoPE's table (H3Transformer.swift:64-78): n_freq checkpoint frequencies
 * shared by the t, h, w axes; pair p uses axis p / n_freq and
 * inv_freq[p % n_freq]. Writes 3*n_freq entries; returns the count. */
int h3hip_rope_pairs_h3(const float* inv_freq, int32_t n_freq, int32_t* pair_axis,
                        float* pair_inv_freq);
/* Integer lattice positions: prefix tokens at (0,0,0), video (t, y, x). */
int h3hip_positions_grid(int32_t prefix_len, int32_t frames, int32_t height, int32_t width,
                         float* pos);
/* PackedLayout.positionIds for text | target audio | target video
 * (Sources/H3Foundation/PackedSequence.swift:185-296): float64 [S, 3].
 * Returns S, or H3HIP_EINVAL for an axis smaller than the patch. */
int h3hip_positions_packed(int32_t text_tokens, int32_t audio_t, int32_t latent_t,
                           int32_t latent_h, int32_t latent_w, int32_t patch, double* pos);
/* Landmark frames of AxialTopology.init(geometry:landmarks:)
 * (AxialTopology.swift:82-112): n clamped to [2, frames], evenly spaced with
 * both ends, deduplicated, ascending. Returns the count written to out[frames]. */
int h3hip_landmarks(int32_t frames, int32_t n, int32_t* out);

#ifdef __cplusplus
}
#endif
#endif /* CH3HIP_H */
