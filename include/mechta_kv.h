/*
 * mechta_kv.h -- C ABI of the MI355X-native KV-cache path of mechta (libmechta_kv.so).
 *
 * One handle = the KV store of `layers` full-attention layers of one model instance: K and V per layer, 2 KV heads of
 * head_dim 256, `ctx` positions, f16 (default) or f32. The reference keeps the same data as one K and one V wgpu
 * buffer per layer (engine.rs:493-496, Engine.kv_buf engine.rs:240); here the store owns one HBM allocation and the
 * layout inside it is the library's (see "Layout"). Every device pointer argument is a plain HIP device address;
 * sizes are in elements unless named *_bytes. No call takes or returns framework types.
 *
 * Ordering: every call is enqueued on the handle's HIP stream (mkv_create / mkv_set_stream) and returns without
 * waiting, except mkv_sync, mkv_snapshot (waits for the copy into host memory) and mkv_destroy. One thread per handle
 * at a time, as the reference's engine thread (api/src/lib.rs:46).
 *
 * Errors: 0 = ok, a negative MKV_E_* code otherwise; mkv_last_error() returns the message of the last failure on the
 * calling thread. The reference panics in the same situations (check_ctx engine.rs:28-33, pos + K < ctx
 * quad.rs:278, pending-row asserts engine.rs:682/785/847); here the call is refused and nothing is enqueued.
 *
 * Length: the store records for each layer how many positions hold data (`len`). An append must start at or before
 * len (no holes) and sets len = pos + ntok; attention may read positions < len only; mkv_set_len shrinks len, which
 * is the rollback of rejected MTP drafts (the reference rolls back by starting the next step at pos + na + 1 and
 * overwriting, quad.rs:320, session.rs:396-401: the next append here overwrites the same rows).
 *
 * Layout: per (layer, K|V, kv head) one contiguous plane of ctx*256 elements. f16: K planes are tiled in blocks of 32
 * positions, [pos/32][d/8][pos%32][8]; V planes in groups of 8 positions, [pos/8][d][pos%8]. f32: K [pos/32][d/4]
 * [pos%32][4], V [pos/4][d][pos%4]. These are the operand layouts of the CDNA4 32x32x16 f16 and 32x32x2 f32 MFMAs,
 * so attention streams them with 16-byte loads straight into matrix operands. mkv_read_rows / mkv_write_rows convert to and from the reference's position-major
 * layout ([pos][kvh][256], kv.wgsl:7-8), e.g. for the reference's root files.
 */
#ifndef MECHTA_KV_H
#define MECHTA_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mkv_store mkv_t;

/* KV formats: KvFormat::{F16, F32} (engine.rs:49-68); MECHTA_KV=f16|f32 */
#define MKV_F16 0
#define MKV_F32 1

/* which cache of a layer */
#define MKV_K 0
#define MKV_V 1

#define MKV_OK 0
#define MKV_E_ARG (-1)   /* bad argument: null pointer, ntok out of range, unknown format */
#define MKV_E_CTX (-2)   /* ctx not a multiple of 1024 in [4096, 262144] (check_ctx, engine.rs:28-33) */
#define MKV_E_POS (-3)   /* position range outside the store or past the written length */
#define MKV_E_LAYER (-4) /* layer index out of range */
#define MKV_E_SIZE (-5)  /* byte count of a snapshot buffer does not match mkv_snapshot_bytes */
#define MKV_E_HIP (-6)   /* HIP runtime failure (message in mkv_last_error) */
#define MKV_E_NOMEM (-7) /* device allocation failed */
#define MKV_E_FMT (-8)   /* operation not available for this KV format, or a root file that does not fit the store */
#define MKV_E_IO (-9)    /* root file missing, unreadable, truncated or not a root file */

#define MKV_CTX_MIN 4096   /* engine.rs:22 */
#define MKV_CTX_MAX 262144 /* engine.rs:23 */
#define MKV_KV_HEADS 2
#define MKV_Q_HEADS 16
#define MKV_HEAD_DIM 256
#define MKV_PREFILL_MAX 512 /* tokens per prefill block, NB (engine.rs:18) */

/* Bytes of one K or V cache of one layer for ctx positions: ctx x 512 elements of the format, as the reference's
 * KvFormat::buffer_bytes_for (engine.rs:64-65); 0 for a bad format. */
size_t mkv_buffer_bytes(int ctx, int fmt);
/* Device bytes mkv_create(layers, ctx, fmt) allocates: the planes (exactly 2 x layers x mkv_buffer_bytes(ctx, fmt):
 * the blocked layout holds ctx x 512 elements per layer and K|V with no padding, ctx being a multiple of 1024), 64 KiB
 * of slack past the last plane, the decode partials (2 kv heads x 32 rows x min(ctx / 64 + 2, 256) splits x 1,040
 * bytes) and the prefill partials (68,157,440 bytes: 2 kv heads x 4,096 (token, split) pairs x 8 heads x 1,040
 * bytes). 0 for arguments mkv_create refuses. The reference's memory check sizes the same cache as
 * 2 x layers x buffer_bytes_for(ctx) (memcheck.rs:110-111). Not included: the no-allocation entry point's scratch
 * (mkv_noalloc_scratch_bytes), a file-scope device array every GPU holds once the library is loaded, whatever the
 * number of stores. */
size_t mkv_store_bytes(int layers, int ctx, int fmt);
/* Bytes of the device scratch of mkv_append_decode_noalloc, held on every GPU the library runs on until the process
 * ends (16,506,880). No counterpart in the reference: for memory checks that must count it. */
size_t mkv_noalloc_scratch_bytes(void);

/* Allocates the store: layers x {K, V} x 2 heads x ctx x 256 elements, zero filled, and the split-K workspaces.
 * Replaces the per-layer KV buffer allocation (engine.rs:493-496) with the ctx check of check_ctx (engine.rs:28-33).
 * stream: a hipStream_t (NULL = the default stream). */
int mkv_create(mkv_t** out, int layers, int ctx, int fmt, void* stream);
/* Frees everything (waits for the stream first). Replaces dropping the Engine's buffers. */
int mkv_destroy(mkv_t* h);
/* Changes the stream later calls are enqueued on. */
int mkv_set_stream(mkv_t* h, void* stream);
/* Waits for all work enqueued by this handle (the reference's device.poll(Wait)). */
int mkv_sync(mkv_t* h);
/* Message of the last failed call on this thread ("" if none). */
const char* mkv_last_error(void);

/* Store geometry and the recorded length of a layer. */
int mkv_info(const mkv_t* h, int* layers, int* ctx, int* fmt);
int mkv_len(const mkv_t* h, int layer, int* len);

/* K/V append of ntok (1..512) tokens at positions pos..pos+ntok-1 of one layer.
 *   k_normed: [ntok][2][256] f32, K after the k RMSNorm, before RoPE (device);
 *   v:        [ntok][512] f32 (device);
 *   rope_tab: [ntok][64] f32, rope_table(pos + t) = [cos th_0..th_31 | sin th_0..th_31] (device).
 * K gets NEOX RoPE on dims 0..63, pairs (i, i+32), computed as a*c - b*s / a*s + b*c with every product and sum
 * rounded to f32 (no FMA), then f32->f16 round to nearest even (f16 store) or stored as is (f32 store).
 * Replaces kv_rope / kv_rope2 + kv_copy (kv.wgsl:19-42) and rope / rope2 + copy (ops.wgsl:141-162, 275-286). */
int mkv_append(mkv_t* h, int layer, int pos, int ntok, const float* k_normed, const float* v, const float* rope_tab);

/* Sets the length of every layer to len (len <= each layer's current length): rollback of rejected drafts. */
int mkv_set_len(mkv_t* h, int len);

/* Decode attention of ntok (1..4) query tokens of one layer, GQA 8:1, split-K over positions.
 *   q: [ntok][16][256] f32 (device), after q RoPE; token t sees positions [start, n + t) (n = pos + 1 of token 0);
 *   out: [ntok][16][256] f32 (device) = softmax(q.k * scale) . v per head;
 *   gate_src: NULL, or qf [ntok][16][512] f32 (device, q | gate interleaved per head): then
 *             out = attention * sigmoid(qf[h*512 + 256 + d]) (attn_gate, ops.wgsl:171-177).
 * Requires n + ntok - 1 <= len(layer). Replaces attn_fd (ops.wgsl:310-394), q_dmx + attn_dmx2 (dmx.rs:19-138) and
 * attn_fd_combine (ops.wgsl:523-538). f16 store: Q and P rounded to f16 for the matrix units, f32 sums (as attn_dmx);
 * f32 store: f32-class throughout (as attn_fd; products on the f16 matrix units from f32 operands split into f16
 * hi + lo, within 1e-5 of exact f32). */
int mkv_decode(mkv_t* h, int layer, const float* q, int ntok, int n, int start, float scale, float* out,
               const float* gate_src);

/* Append + decode of the same ntok tokens in one launch sequence: mkv_append(layer, n - 1, ntok, ...) followed by
 * mkv_decode(layer, q, ntok, n, start, ...). Same results as the two calls. */
int mkv_append_decode(mkv_t* h, int layer, int n, int ntok, const float* k_normed, const float* v,
                      const float* rope_tab, const float* q, int start, float scale, float* out,
                      const float* gate_src);

/* mkv_decode / mkv_append_decode with the gated attention written as f16, the form the reference's 4-token verify
 * (quad.rs:125) and its 2-token step with f16 activations (engine.rs:1103) hand to the f16 attn_output matvec:
 * attn_gate16 (ops.wgsl:296-300), out16[t][h][d] = f16(attention * sigmoid(qf[h*512 + 256 + d])), rounded to nearest
 * even (pack2x16float), as f16 bit patterns, [ntok][16][256] (device; the reference's [ntok][4096] halves).
 * gate_src is required (MKV_E_ARG if NULL); every other argument and check as the f32 entry points. */
int mkv_decode_g16(mkv_t* h, int layer, const float* q, int ntok, int n, int start, float scale, uint16_t* out16,
                   const float* gate_src);
int mkv_append_decode_g16(mkv_t* h, int layer, int n, int ntok, const float* k_normed, const float* v,
                          const float* rope_tab, const float* q, int start, float scale, uint16_t* out16,
                          const float* gate_src);

/* mkv_append_decode with no allocation of any kind: for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. Same arguments, results
 * bit-identical to mkv_append_decode; the split-K partials go to a scratch array of the library (16,506,880 bytes per
 * GPU, held until the process ends) instead of the handle's workspace. Limit: at most 248 splits (every decode plan of
 * 1..4 tokens fits; MKV_E_SIZE otherwise, nothing enqueued). The scratch is shared by every handle on one GPU: calls
 * that overlap on one GPU (on different streams, or from different handles without ordering) race, so a caller with
 * two handles on one GPU (e.g. the 10-layer store and the MTP layer's) must order their calls on one stream. The
 * scratch's address is resolved by mkv_create with the device current (or by the first call, with the handle's device
 * current); MKV_E_HIP when it cannot be. The handle's trace (mkv_trace) records nothing for this call: taking trace
 * events may allocate. */
int mkv_append_decode_noalloc(mkv_t* h, int layer, int n, int ntok, const float* k_normed, const float* v,
                              const float* rope_tab, const float* q, int start, float scale, float* out,
                              const float* gate_src);

/* Causal prefill attention of T (1..512) tokens of one layer: token t sees positions [start, n + t).
 *   q: [T][16][256] f32 (device); out: [T][16][256] f32 (device); gate_src as mkv_decode ([T][16][512]).
 * Requires n + T - 1 <= len(layer). Replaces q_f16 + attn_fa_mx + attn_fd_combine (fa_mx.wgsl:19-115, 313-319;
 * engine.rs:1215-1236) and attn_fa / attn_fd4 for the f32 store (ops.wgsl:540-651, 694-778). */
int mkv_prefill(mkv_t* h, int layer, const float* q, int T, int n, int start, float scale, float* out,
                const float* gate_src);

/* Prefix-cache snapshot of positions [0, p) of every layer (the KV part of read_root / write_root,
 * engine.rs:782-823). The byte image is the store's own layout, block-rounded; restore into a store of the same
 * layers / format (any ctx >= p) gives back bit-identical positions [0, p) and sets every layer's length to p.
 * host: pinned host memory (hipHostMalloc) of exactly mkv_snapshot_bytes(h, p) bytes; pageable memory is refused with
 * MKV_E_ARG before anything is enqueued.
 * mkv_snapshot waits until the copy has landed in host memory; mkv_restore returns when the copy is enqueued
 * (the host buffer must stay valid until mkv_sync). */
size_t mkv_snapshot_bytes(const mkv_t* h, int p);
int mkv_snapshot(mkv_t* h, int p, void* host, size_t bytes);
int mkv_restore(mkv_t* h, int p, const void* host, size_t bytes);

/* Conversion to / from the reference's position-major layout for positions [p0, p1) of one layer's K or V:
 * dst/src (device) hold (p1 - p0) x 512 elements in the store's element type (f16 bit patterns or f32),
 * element (pos, kvh, d) at (pos - p0)*512 + kvh*256 + d -- the words read_root writes for that range
 * (engine.rs:784-802). mkv_write_rows extends the layer's length to p1 if p0 <= len. */
int mkv_read_rows(mkv_t* h, int layer, int which, int p0, int p1, void* dst);
int mkv_write_rows(mkv_t* h, int layer, int which, int p0, int p1, const void* src);

/* GPU time spans of the path's kernels: the counterpart of the reference's GPU timestamp spans around the attention
 * groups attn.kv_write / attn.core / attn.merge (MECHTA_TRACE=2; gpu/src/lib.rs:297-341, engine.rs:1274-1299).
 * While tracing is on, every kernel launch of the handle is bracketed by two HIP events on the handle's stream.
 * mkv_trace(h, 1) starts (and clears), mkv_trace(h, 0) stops; mkv_trace_read waits for the stream and returns, per
 * span, the summed kernel milliseconds and the number of launches since tracing started. */
#define MKV_SPAN_KV_WRITE 0 /* append kernels */
#define MKV_SPAN_CORE 1     /* split-K decode and prefill attention kernels */
#define MKV_SPAN_MERGE 2    /* merge of the split-K partials (+ gate) */
#define MKV_SPANS 3
int mkv_trace(mkv_t* h, int enable);
int mkv_trace_read(mkv_t* h, double* ms /*[MKV_SPANS]*/, long* count /*[MKV_SPANS]*/);

/* rope_table(pos) on the host (engine.rs:108-114): tab[0..32) = cos, tab[32..64) = sin of th_i, th_0 = pos,
 * th_{i+1} = th_i * 1e7^(-2/64), all in f32. */
int mkv_rope_table(int pos, float* tab);

/* RoPE table on the device: rows [pos][64] of rope_table (the f32 values mkv_rope_table computes on the host, so
 * the bits are the same) for every position [0, ctx) of the store, built on the first call (a synchronous upload:
 * call it once before any graph capture) and kept until mkv_destroy. *tab points at row pos; rows pos + 1 .. follow
 * it. Use it as the rope_tab of mkv_append / mkv_append_decode instead of uploading tables per step (the reference
 * writes a table per step, engine.rs:626-630). */
int mkv_rope_table_dev(mkv_t* h, int pos, const float** tab);

/* The q/k producer in front of the append, one launch for the reference's rmsnorm of q, rmsnorm of k and rope2 of
 * q (quad.rs:113-115, engine.rs:1210-1212; ops.wgsl:27-57 with the qn / kn uniforms of quad.rs:50, ops.wgsl:275-286)
 * for ntok tokens at positions pos .. pos + ntok - 1:
 *   qf: [ntok][16][512] f32 (each head's 256 q values, then its 256 gate values: the attn_q matvec output);
 *   kb: [ntok][2][256] f32 (the attn_k matvec output); q_norm_w, k_norm_w: [256] (attn_q_norm / attn_k_norm);
 *   eps: the RMSNorm epsilon (1e-6, engine.rs:12);
 *   q_out: [ntok][16][256] = rope2(rmsnorm(q)), the q of mkv_decode / mkv_append_decode / mkv_prefill;
 *   kn_out: [ntok][2][256] = rmsnorm(k), the k_normed of mkv_append / mkv_append_decode.
 * The sum of squares follows the reference's 256-thread tree reduction; square root and division are correctly
 * rounded; no product is contracted into an FMA. The RoPE rows come from mkv_rope_table_dev. */
int mkv_qk_norm_rope(mkv_t* h, int pos, int ntok, const float* qf, const float* kb, const float* q_norm_w,
                     const float* k_norm_w, float eps, float* q_out, float* kn_out);

/* Root files: the prefix cache across sessions on disk (write_root_file / read_root_file, session.rs:92-129), byte for
 * byte the reference's container, so the files are interchangeable with its:
 *   "MECHTA-ROOT-1\n", u64 p, u64 ns, u64 nk, p x u32 tokens, ns SSM vectors, ns conv vectors, nk x (K vector,
 *   V vector); a vector is a u64 word count followed by that many 32-bit words; every number little-endian.
 * The KV vectors are the words read_root gathers for the attention layers (engine.rs:784-802): positions [0, p)
 * position-major ([pos][kvh][256]), f32 values or pairs of f16 bits, p*512 (f32) or p*256 (f16) words; nk is the
 * store's layer count. The SSM / conv vectors are the caller's model state (the DeltaNet layers of the reference)
 * and pass through as opaque 32-bit words.
 *
 * mkv_root_key: FNV-1a 64 of the tokens' little-endian bytes (root_key, session.rs:62-66), the key in the file name.
 * mkv_root_save: gathers positions [0, p) of every layer (waits for the copy into host memory), then writes
 *   path + ".tmp" and renames it to path (as write_root_file). With background != 0 the file write runs on a thread
 *   of the handle and mkv_root_save returns once the words are in host memory; mkv_root_wait joins it and returns
 *   its result (a later mkv_root_save or mkv_destroy joins it too). tokens: p entries; ssm[i], conv[i]: host arrays
 *   of ssm_words[i], conv_words[i] words (i < ns), copied before the call returns.
 * mkv_root_info: p, ns and nk of a file, the KV vectors' word count, and (arrays of at least max_ns entries, or
 *   NULL) the SSM / conv vectors' word counts; checks that the file holds every word its header announces.
 * mkv_root_load: puts a root file into the store: every layer's positions [0, p) (the length becomes p) from the KV
 *   vectors, and the tokens / state vectors into the caller's arrays (NULL to skip; sizes from mkv_root_info).
 *   Refused (MKV_E_FMT, store unchanged) unless nk == layers, p <= ctx and the KV word count matches the format.
 *   Returns when the store holds the data. */
uint64_t mkv_root_key(const uint32_t* tokens, size_t n);
int mkv_root_save(mkv_t* h, const char* path, int p, const uint32_t* tokens, int ns, const float* const* ssm,
                  const uint64_t* ssm_words, const float* const* conv, const uint64_t* conv_words, int background);
int mkv_root_wait(mkv_t* h);
int mkv_root_info(const char* path, int* p, int* ns, int* nk, uint64_t* kv_words, uint64_t* ssm_words,
                  uint64_t* conv_words, int max_ns);
int mkv_root_load(mkv_t* h, const char* path, uint32_t* tokens, float* const* ssm, float* const* conv);

/* Root-file policy of the reference's session (session.rs:61-90):
 * MKV_ROOT_MIN: a root is taken only for a system prompt of at least this many tokens (ROOT_MIN, session.rs:90).
 * mkv_root_path: the file name of a root, "<dir>/root-<f16|f32>-<model key>-<token key>.bin" (root_file,
 *   session.rs:68-73), the keys as 16 lower-case hex digits: the model key is FNV-1a 64 of the model path's bytes, each
 *   byte taken as one u32 token (root_key over model_path().bytes().map(u32::from)), the token key mkv_root_key of the
 *   prompt. Writes at most cap bytes with the terminating NUL; returns the name's length (not counting the NUL), or
 *   MKV_E_ARG (NULL argument, bad format) / MKV_E_SIZE (cap too small, nothing written past out[cap - 1]).
 * mkv_root_prune: keeps the `keep` (at least 1) most recently modified files of `dir` whose names start with
 *   "root-<fmt>-" and end with ".bin", and removes the others (prune_roots, session.rs:75-84; MECHTA_ROOTS defaults to
 *   6 there). Returns the number removed; 0 when the directory cannot be read (the reference gives up silently too).
 * mkv_root_touch: sets a root file's modification time to now, so the pruning keeps it (touch, session.rs:86-88);
 *   0, or MKV_E_IO when the file cannot be opened. */
#define MKV_ROOT_MIN 2048
int mkv_root_path(char* out, size_t cap, const char* dir, int fmt, const char* model_path, const uint32_t* tokens,
                  size_t n);
int mkv_root_prune(const char* dir, int fmt, int keep);
int mkv_root_touch(const char* path);

#ifdef __cplusplus
}
#endif
#endif
