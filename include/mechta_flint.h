/* mechta_flint.h -- the Flint model's KV-cache path (sliding-window ring KV with per-head attention sinks) on one
 * MI355X, in the same library as mechta_kv.h (libmechta_kv.so). Error codes are the MKV_E_* of mechta_kv.h and the
 * message of a failed call is in mkv_last_error().
 *
 * Flint (engine/crates/mechta/src/flint.rs:12-32) has attention in every layer: 32 query heads and 4 KV heads of
 * head_dim 128 (GQA 8:1). A sliding layer keeps its K/V in a ring of 1024 rows (row = position % 1024, RING_SWA,
 * flint.rs:26) and a token sees the current position and the 512 before it (WINDOW = 513, flint.rs:23); a full layer
 * keeps ctx rows (no wrap) and sees every earlier position. Attention scores are scaled by 1/sqrt(128), and each
 * query head's sink logit joins the softmax maximum and sum but not the output (flint_attn.wgsl:1-8, 241-257).
 *
 * Layout: per (layer, K|V, kv head) one plane of rows x 128 elements. f32: K [row/32][d/4][row%32][4], V [row/4][d]
 * [row%4]; f16: K [row/32][d/8][row%32][8], V [row/8][d][row%8] -- the operand layouts of the CDNA4 matrix
 * instructions. Attention arithmetic is f32-class, as the reference's f32: products run on the f16 matrix units with
 * f32 operands split into f16 hi + lo (hi.hi + hi.lo + lo.hi, f32 accumulation; within 1e-5 of exact f32). mfl_read_rows /
 * mfl_write_rows convert to and from the reference's row layout [row][kvh][128] (flint_attn.wgsl:3, kv_put).
 *
 * All calls are ordered on the handle's stream; device pointers are plain HIP device addresses. A decode of 1-2 tokens
 * over a short span (up to 384 positions on an f32 cache, 512 on an f16 one) merges its split partials in the kernel, through per-kv-head arrival counters the handle keeps: two such
 * decodes of one handle must not run at once, so keep every call of a handle on one stream (mfl_set_stream moves them
 * all).
 */
#ifndef MECHTA_FLINT_H
#define MECHTA_FLINT_H

#include "mechta_kv.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mfl_store mfl_t;

#define MFL_Q_HEADS 32
#define MFL_KV_HEADS 4
#define MFL_HEAD_DIM 128
#define MFL_RING_SWA 1024 /* flint.rs:26 */
#define MFL_WINDOW 513    /* flint.rs:23 */
#define MFL_BLOCK_MAX 512 /* tokens of a prefill block, NB (flint.rs:28) */

/* Allocates the K/V of `layers` layers, zero filled: layer l holds 1024 rows if sliding[l] != 0, else ctx rows.
 * ctx: a multiple of 1024 in [1024, 262144]; fmt: MKV_F32 (the reference's default) or MKV_F16 (MECHTA_FLINT_KV=f16,
 * flint.rs:72-90). Replaces the kc / vc buffers of Flint::new (flint.rs:227-232). The handle also holds the
 * attention's split partials, 34.6 MB, allocated here, so attention calls never allocate. */
int mfl_create(mfl_t** out, int layers, int ctx, int fmt, const unsigned char* sliding, void* stream);
int mfl_destroy(mfl_t* h);
int mfl_set_stream(mfl_t* h, void* stream);
int mfl_sync(mfl_t* h);
/* Rows of layer `layer` (1024 or ctx). */
int mfl_rows(const mfl_t* h, int layer, int* rows);

/* Host RoPE table of position pos: [cos th_0..th_63 | sin th_0..th_63], th_0 = pos, th_{i+1} = th_i * base^(-2/128),
 * all in f32 (rope_table, flint.rs:61-68; ggml_rope_cache_init). */
int mfl_rope_table(int pos, float base, float* tab /* [128] */);
/* NEOX RoPE of ntok tokens x heads rows of 128 (pairs (i, i + 64)): out = x rotated by the table row of its token.
 * x, out: [ntok][heads][128] (device, may alias); tab: [ntok][128] (device). Replaces rope_neox / rope_neox_n
 * (flint_attn.wgsl:24-31, 46-53). */
int mfl_rope(mfl_t* h, int ntok, int heads, const float* x, const float* tab, float* out);

/* Writes the K (after RoPE on RoPE layers) and V rows of ntok tokens at positions pos0 .. pos0 + ntok - 1 to rows
 * (pos0 + t) % rows of the layer; f16 store: f32 -> f16 round to nearest even. k, v: [ntok][4][128] f32 (device).
 * Replaces kv_write / kv_write_n (flint_attn.wgsl:34-38, 56-61). A sliding layer's block must not overwrite a row a
 * token of the same block still sees (ntok <= 1024 - 512). */
int mfl_append(mfl_t* h, int layer, int pos0, int ntok, const float* k, const float* v);

/* Attention of ntok tokens at positions pos0 .. pos0 + ntok - 1 whose K/V rows are already written: token t sees the
 * positions [lo_t, pos0 + t], lo_t = max(0, pos0 + t + 1 - 513) on sliding layers, 0 on full layers.
 *   q: [ntok][32][128] f32 (device, after RoPE on RoPE layers); sinks: [32] f32 (device, attn_sinks) or NULL;
 *   out: [ntok][32][128] f32 (device) = softmax with the sink of q.k / sqrt(128), times V.
 * ntok = 1 replaces attn_fd + attn_fd_merge (flint_attn.wgsl:172-257), ntok > 1 (<= 512) attn_pf
 * (flint_attn.wgsl:63-170). */
int mfl_attend(mfl_t* h, int layer, int pos0, int ntok, const float* q, const float* sinks, float* out);

/* Conversion to / from the reference's row layout for rows [r0, r1) of a layer's K or V (which = MKV_K / MKV_V):
 * dst/src (device) hold (r1 - r0) x 512 elements [row][kvh][128] of the store's element type (f32, or f16 bits).
 * With these a root is read_root / write_root (flint.rs:320-331): rows [0, p) of full layers, the whole ring of
 * sliding ones. */
int mfl_read_rows(mfl_t* h, int layer, int which, int r0, int r1, void* dst);
int mfl_write_rows(mfl_t* h, int layer, int which, int r0, int r1, const void* src);

/* Photo of the sliding rings (photograph / restore_photo, flint.rs:308-316): device copies of every sliding layer's
 * K and V planes into / from a device buffer the handle owns (allocated on the first photo). */
int mfl_photo(mfl_t* h);
int mfl_restore_photo(mfl_t* h);

#ifdef __cplusplus
}
#endif
#endif
