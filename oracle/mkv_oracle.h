/*
 * mkv_oracle.h -- CPU restatement of mechta's KV-cache path (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the checker for the HIP path in mechta_amd/: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it. The product library never links or calls it.
 *
 * Every function follows a named reference file:line of ssomenzi/mechta (Rust + WGSL). Layout conventions are the
 * reference's own: the cache of one layer is position-major, element (pos, kvh, d) at pos*512 + kvh*256 + d
 * (wgsl/ops.wgsl:165, wgsl/kv.wgsl:7-8); f16 caches are arrays of IEEE binary16 bit patterns (uint16_t), two per
 * u32 word in the reference's packing (pack2x16float: low half = even element), which is the same byte order.
 *
 * Fixed conventions where WGSL leaves the result open (both fixed by the task statement):
 *   - pack2x16float and f16(x) round to nearest even (orc_f32_to_f16);
 *   - a*b - c*d in kv_src is NOT fused: each product is rounded to f32, then the sum (build with -ffp-contract=off).
 *
 * Parity pinning (what checks each function independently of its own formula) is listed in tests/test_oracle.py.
 */
#ifndef MKV_ORACLE_H
#define MKV_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define ORC_KVH 2
#define ORC_H 16
#define ORC_D 256
#define ORC_ROW (ORC_KVH * ORC_D) /* 512 elements per position */

/* IEEE-754 binary32 -> binary16, round to nearest even (WGSL pack2x16float as fixed by the north star). */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_n(const float* x, uint16_t* y, int64_t n);

/* rope_table(pos): [cos th_0..th_31 | sin th_0..th_31], th_0 = pos, th_{i+1} = th_i * 1e7^(-2/64) in f32.
 * engine.rs:108-114 */
void orc_rope_table(int32_t pos, float tab[64]);

/* K/V append of ntok tokens at positions pos..pos+ntok-1 into one layer's cache.
 * fmt 0 = f16 (kc/vc are uint16_t*), 1 = f32 (float*).
 * kn: [ntok][2][256] normed K before RoPE; v: [ntok][512]; tab: [ntok][64] (rope_table of pos+t).
 * f16: kv.wgsl:19-42 (kv_src, kv_row, kv_rope2 with flag = 2, kv_copy).
 * f32: ops.wgsl:141-145 (copy), ops.wgsl:275-286 (rope2). */
void orc_append(int fmt, void* kc, void* vc, int pos, int ntok, const float* kn, const float* v, const float* tab);

/* Decode attention with the semantics of attn_fd + attn_fd_combine (ops.wgsl:310-394, 523-538): per token t the
 * keys [start, n + t), exact f32 softmax per block of `bb` positions (128 in the reference), partials merged with the
 * log-sum-exp formula. q: [ntok][16][256] f32; out: [ntok][16][256] f32. fmt as orc_append. */
void orc_attn_fd(int fmt, const void* kc, const void* vc, const float* q, int ntok, int n, int start, float scale,
                 int bb, float* out);

/* Decode attention with the semantics of q_dmx + attn_dmx2 + attn_fd_combine (dmx.rs:19-138, ops.wgsl:523-538):
 * Q rounded to f16, S = Q.K^T with f32 sums, keys in tiles of 64 inside chunks of `ch` positions, lazy reference
 * max (moves when first or when the tile max exceeds it by more than 8), P = f16(exp(s - m)), l += f32(P),
 * O += P.V. Row r = t*8 + head sees keys < n + t. f16 cache only. */
void orc_attn_dmx(const uint16_t* kc, const uint16_t* vc, const float* q, int ntok, int n, float scale, int ch,
                  float* out);

/* Prefill attention with the semantics of q_f16 + attn_fa_mx + attn_fd_combine (fa_mx.wgsl:19-115, 313-319;
 * engine.rs:1215-1236): Q and K in f16, S with f32 sums, exact online max per 64-key tile, P in f32, V from the f16
 * cache, chunks of `ch` = FA_CH = 2048 keys starting at `start`. Token t (0-based in the block) sees keys
 * [start, n + t). q: [T][16][256]. Only the tokens listed in sel[0..nsel) are computed (sel = NULL: all T);
 * out: [nsel][16][256]. f16 cache only. */
void orc_attn_fa_mx(const uint16_t* kc, const uint16_t* vc, const float* q, int T, int n, int start, float scale,
                    int ch, const int* sel, int nsel, float* out);

/* f32-cache prefill (attn_fa, ops.wgsl:540-651): exact f32 math; same result contract as orc_attn_fd per token. */
void orc_attn_fa_f32(const float* kc, const float* vc, const float* q, int T, int n, int start, float scale,
                     const int* sel, int nsel, float* out);

/* Small-block prefill (attn_fd4 + attn_fd_combine, ops.wgsl:694-778, 523-538; dispatched for blocks of fewer than 64
 * tokens, engine.rs:1237-1241, with the uniforms of engine.rs:919-921: extra = 0, flag = PREFILL_BLOCK = 64): f32 Q
 * against the cache (f16 values widened exactly), token t of the block sees [0, n + t), per block of bl positions an
 * exact online max over tiles of 64, blocks merged with the log-sum-exp formula. q, out: [T][16][256]. */
void orc_attn_fd4(int fmt, const void* kc, const void* vc, const float* q, int T, int n, float scale, int bl,
                  float* out);

/* Output gate, attn_gate (ops.wgsl:171-177): out[t][h*256+d] = att[t][h*256+d] * sigmoid(qf[t][h*512+256+d]). */
void orc_gate(const float* att, const float* qf, int ntok, float* out);
void orc_gate16(const float* att, const float* qf, int ntok, uint16_t* out);

/* Threads used by the OpenMP loops (for the CPU-baseline report). */
int orc_threads(void);

/* rmsnorm of `rows` rows of 256 values (row r at x + r*step) with weight w (ops.wgsl:27-57, the q/k norm uniforms
 * of quad.rs:50): the reference's 256-thread tree reduction, correctly rounded sqrt and division. y: [rows][256]. */
void orc_rmsnorm_rows(const float* x, int rows, int step, const float* w, float eps, float* y);
/* q/k producer of ntok tokens (quad.rs:113-115): q norm + rope2 (ops.wgsl:275-286) into q_out [ntok][16][256],
 * k norm into kn_out [ntok][2][256]; qf: [ntok][16][512] (q | gate), kb: [ntok][2][256], tab: [ntok][64]. */
void orc_qk_norm_rope(const float* qf, const float* kb, int ntok, const float* q_w, const float* k_w, float eps,
                      const float* tab, float* q_out, float* kn_out);

#ifdef __cplusplus
}
#endif
#endif
