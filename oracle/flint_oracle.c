/*
 * flint_oracle.c -- CPU restatement of the Flint model's KV path (flint_attn.wgsl, flint.rs).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path's mfl_* calls (tests/). Nothing in mechta_amd/ links, loads
 * or calls this file. Built into libmkv_oracle.so by oracle/build.py (gcc -O3 -fopenmp -ffp-contract=off).
 *
 * Caches here use the reference's layout: per layer a K and a V array of `ring` rows x 512 elements (row = position %
 * ring, 4 KV heads x 128), f32 values or f16 bit patterns (kv_put of the f16 block, flint.rs:83-90: pack2x16float).
 *
 * Parity pinning (tests/test_oracle.py): the RoPE table against float64 cos/sin of the f32 angle recurrence; RoPE
 * against float64 rotation and the identity at position 0; the writes against numpy's float16 cast and the ring
 * index; both attentions against a float64 textbook softmax with the sink term, the sink limits (very negative: plain
 * softmax; very large: zero output), the window (rows outside it changed, output unchanged), and attn_pf of one token
 * against attn_fd.
 */
#include "flint_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "mkv_oracle.h"

#define FL_H 32
#define FL_KVH 4
#define FL_D 128
#define FL_ROW (FL_KVH * FL_D)
#define NEG_BIG (-3.0e38f) /* flint_attn.wgsl:128, 202 */

/* rope_table (flint.rs:61-68): scale = base^(-2/128) in f32, theta_0 = pos, theta_{i+1} = theta_i * scale. */
void orc_fl_rope_table(int pos, float base, float* tab) {
    float scale = powf(base, -2.0f / (float)FL_D);
    float theta = (float)pos;
    for (int i = 0; i < FL_D / 2; i++) {
        tab[i] = cosf(theta);
        tab[FL_D / 2 + i] = sinf(theta);
        theta = theta * scale;
    }
}

/* rope_neox_n (flint_attn.wgsl:46-53): pair (i, i + 64) of each 128-row; rows = ntok * heads, row r uses table row
 * r / heads. */
void orc_fl_rope(int ntok, int heads, const float* x, const float* tab, float* out) {
    for (int r = 0; r < ntok * heads; r++) {
        const float* tb = tab + (size_t)(r / heads) * FL_D;
        const float* a = x + (size_t)r * FL_D;
        float* o = out + (size_t)r * FL_D;
        for (int i = 0; i < 64; i++) {
            float x0 = a[i], x1 = a[i + 64];
            float p = x0 * tb[i], q = x1 * tb[64 + i];
            float u = x0 * tb[64 + i], w = x1 * tb[i];
            o[i] = p - q;
            o[i + 64] = u + w;
        }
    }
}

static float kv_elem(int fmt, const void* c, size_t i) {
    if (fmt == 1) return ((const float*)c)[i];
    return orc_f16_to_f32(((const uint16_t*)c)[i]);
}

/* kv_write_n (flint_attn.wgsl:56-61): token t of the block into row (pos0 + t) % ring. */
void orc_fl_kv_write(int fmt, void* kc, void* vc, int ring, int pos0, int n, const float* k, const float* v) {
    for (int t = 0; t < n; t++) {
        size_t r = (size_t)((pos0 + t) % ring) * FL_ROW;
        for (int i = 0; i < FL_ROW; i++) {
            if (fmt == 1) {
                ((float*)kc)[r + i] = k[(size_t)t * FL_ROW + i];
                ((float*)vc)[r + i] = v[(size_t)t * FL_ROW + i];
            } else {
                ((uint16_t*)kc)[r + i] = orc_f32_to_f16(k[(size_t)t * FL_ROW + i]);
                ((uint16_t*)vc)[r + i] = orc_f32_to_f16(v[(size_t)t * FL_ROW + i]);
            }
        }
    }
}

/* dot of 4 consecutive products, the WGSL dot() of two vec4 (flint_attn.wgsl:197-199). */
static float dot4(const float* a, const float* b) {
    float p0 = a[0] * b[0], p1 = a[1] * b[1], p2 = a[2] * b[2], p3 = a[3] * b[3];
    return ((p0 + p1) + p2) + p3;
}

#define FD_CH 256

/* attn_fd + attn_fd_merge (flint_attn.wgsl:172-257) of one token: q [32][128]; positions lo .. lo + n - 1 at rows
 * pos % ring; pieces of 256 positions: per (head, piece) max, sum of exp and exp-weighted V; then the merge with the
 * sink. out [32][128]. sinks may be NULL (no sink term). */
void orc_fl_attn_fd(int fmt, const void* kc, const void* vc, int ring, const float* q, int lo, int n,
                    const float* sinks, float* out) {
    const float scale = 1.0f / sqrtf(128.0f);
    int nch = (n + FD_CH - 1) / FD_CH;
    float* pm = (float*)malloc(sizeof(float) * FL_H * nch);
    float* pl = (float*)malloc(sizeof(float) * FL_H * nch);
    float* pa = (float*)malloc(sizeof(float) * FL_H * nch * FL_D);
    float* s = (float*)malloc(sizeof(float) * FD_CH);
    for (int h = 0; h < FL_H; h++) {
        int g = h / 8;
        const float* qh = q + (size_t)h * FL_D;
        for (int ch = 0; ch < nch; ch++) {
            int j0 = ch * FD_CH, nj = n - j0 < FD_CH ? n - j0 : FD_CH;
            float mm = NEG_BIG;
            for (int j = 0; j < FD_CH; j++) {
                if (j < nj) {
                    size_t k0 = (size_t)((lo + j0 + j) % ring) * FL_ROW + (size_t)g * FL_D;
                    float acc = 0.0f;
                    for (int e = 0; e < FL_D; e += 4) {
                        float kk[4] = {kv_elem(fmt, kc, k0 + e), kv_elem(fmt, kc, k0 + e + 1),
                                       kv_elem(fmt, kc, k0 + e + 2), kv_elem(fmt, kc, k0 + e + 3)};
                        acc += dot4(qh + e, kk);
                    }
                    s[j] = acc * scale;
                } else {
                    s[j] = NEG_BIG;
                }
                mm = s[j] > mm ? s[j] : mm;
            }
            float sm = 0.0f;
            for (int j = 0; j < FD_CH; j++) {
                float e = s[j] > -1.0e38f ? expf(s[j] - mm) : 0.0f;
                s[j] = e;
                sm += e;
            }
            float* a = pa + ((size_t)h * nch + ch) * FL_D;
            for (int d = 0; d < FL_D; d++) a[d] = 0.0f;
            for (int j = 0; j < nj; j++) {
                size_t v0 = (size_t)((lo + j0 + j) % ring) * FL_ROW + (size_t)g * FL_D;
                for (int d = 0; d < FL_D; d++) a[d] += s[j] * kv_elem(fmt, vc, v0 + d);
            }
            pm[h * nch + ch] = mm;
            pl[h * nch + ch] = sm;
        }
        /* attn_fd_merge */
        float sink = sinks ? sinks[h] : NEG_BIG;
        float mm = sink;
        for (int ch = 0; ch < nch; ch++) mm = pm[h * nch + ch] > mm ? pm[h * nch + ch] : mm;
        float ll = sinks ? expf(sink - mm) : 0.0f;
        float acc[FL_D];
        for (int d = 0; d < FL_D; d++) acc[d] = 0.0f;
        for (int ch = 0; ch < nch; ch++) {
            float w = expf(pm[h * nch + ch] - mm);
            ll += w * pl[h * nch + ch];
            for (int d = 0; d < FL_D; d++) acc[d] += w * pa[((size_t)h * nch + ch) * FL_D + d];
        }
        for (int d = 0; d < FL_D; d++) out[(size_t)h * FL_D + d] = acc[d] / ll;
    }
    free(pm);
    free(pl);
    free(pa);
    free(s);
}

static int lo_di(int pos, int win) { return win > 0 && pos + 1 > win ? pos + 1 - win : 0; }

/* attn_pf (flint_attn.wgsl:63-170, with Q, K, V kept in f32 as attn_source makes it): per (KV head, group of 8
 * tokens), 64-key tiles from the group's first token's window start; exact online softmax per row with the running
 * maximum starting at the sink and the running sum at 1 (its exp); token T sees [lo_T, pos0 + T]. q, out:
 * [n][32][128]. sinks may be NULL (running max -3e38, sum 0). */
void orc_fl_attn_pf(int fmt, const void* kc, const void* vc, int ring, const float* q, int pos0, int n, int win,
                    const float* sinks, float* out) {
    const float scale = 1.0f / sqrtf(128.0f);
    int groups = (n + 7) / 8;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int kvh = 0; kvh < FL_KVH; kvh++)
        for (int gi = 0; gi < groups; gi++) {
            int tb = 8 * gi;
            int last = tb + 7 < n - 1 ? tb + 7 : n - 1;
            int last_pos = pos0 + last;
            int lo = lo_di(pos0 + tb, win);
            int ntile = (last_pos + 64 - lo) / 64;
            float fm[64], fl[64], fc[64];
            float acc[64][FL_D];
            float sc[64][64];
            for (int r = 0; r < 64; r++) {
                fm[r] = sinks ? sinks[8 * kvh + r % 8] : NEG_BIG;
                fl[r] = sinks ? 1.0f : 0.0f;
                for (int d = 0; d < FL_D; d++) acc[r][d] = 0.0f;
            }
            for (int tile = 0; tile < ntile; tile++) {
                int k0 = lo + tile * 64;
                for (int r = 0; r < 64; r++) { /* row r = token tb + r / 8, head 8 kvh + r % 8 */
                    int tk = tb + r / 8;
                    int pt = pos0 + tk, lt = lo_di(pt, win);
                    for (int c = 0; c < 64; c++) {
                        int sp = k0 + c;
                        float v = NEG_BIG;
                        if (tk < n && sp <= last_pos && sp >= lt && sp <= pt) {
                            const float* qr = q + ((size_t)tk * FL_H + 8 * kvh + r % 8) * FL_D;
                            size_t kr = (size_t)(sp % ring) * FL_ROW + (size_t)kvh * FL_D;
                            float a = 0.0f;
                            for (int e = 0; e < FL_D; e += 4) {
                                float kk[4] = {kv_elem(fmt, kc, kr + e), kv_elem(fmt, kc, kr + e + 1),
                                               kv_elem(fmt, kc, kr + e + 2), kv_elem(fmt, kc, kr + e + 3)};
                                a += dot4(qr + e, kk);
                            }
                            v = a * scale;
                        }
                        sc[r][c] = v;
                    }
                }
                for (int r = 0; r < 64; r++) {
                    float mo = fm[r], mx = mo;
                    for (int c = 0; c < 64; c++) mx = sc[r][c] > mx ? sc[r][c] : mx;
                    float sm = 0.0f;
                    for (int c = 0; c < 64; c++) {
                        float w = sc[r][c] > -1.0e38f ? expf(sc[r][c] - mx) : 0.0f;
                        sc[r][c] = w;
                        sm += w;
                    }
                    float cf = expf(mo - mx);
                    fc[r] = cf;
                    fm[r] = mx;
                    fl[r] = fl[r] * cf + sm;
                }
                for (int r = 0; r < 64; r++) {
                    for (int d = 0; d < FL_D; d++) acc[r][d] *= fc[r];
                    for (int c = 0; c < 64; c++) {
                        int sp = k0 + c;
                        if (sp > last_pos || sc[r][c] == 0.0f) continue; /* 0 * v adds nothing (finite v) */
                        size_t vr = (size_t)(sp % ring) * FL_ROW + (size_t)kvh * FL_D;
                        for (int d = 0; d < FL_D; d++) acc[r][d] += sc[r][c] * kv_elem(fmt, vc, vr + d);
                    }
                }
            }
            for (int r = 0; r < 64; r++) {
                int tk = tb + r / 8;
                if (tk >= n) continue;
                float* o = out + ((size_t)tk * FL_H + 8 * kvh + r % 8) * FL_D;
                for (int d = 0; d < FL_D; d++) o[d] = acc[r][d] / fl[r];
            }
        }
}
