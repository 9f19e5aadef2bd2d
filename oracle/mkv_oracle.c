/*
 * mkv_oracle.c -- CPU restatement of mechta's KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path (tests/, __graft_entry__.smoke(), bench.py cpu_baseline).
 * Nothing in mechta_amd/ links, loads or calls this file.
 *
 * Built by oracle/build.py with gcc -O3 -fopenmp -ffp-contract=off (no FMA contraction: the restatement rounds every
 * product and every sum to f32, the convention fixed for the reference's kv_src and dot products).
 *
 * Parity pinning: tests/test_oracle.py checks every function here against an independent computation
 * (numpy's float16 cast, float64 textbook softmax attention, closed-form special cases, invariants); no function is
 * "parity unpinned" except where that file says so.
 */
#include "mkv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define NEG_BIG (-3.0e38f) /* the reference's "minus infinity" (ops.wgsl:381, dmx.rs:48) */

/* ---------------------------------------------------------------- f16 ---------------------------------------- */

/* IEEE-754 round to nearest even, written from the format definition: 1 sign, 5 exponent (bias 15), 10 fraction
 * bits; results below 2^-14 are subnormal (step 2^-24); |x| >= 65520 rounds to infinity; NaN stays NaN (quiet). */
uint16_t orc_f32_to_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    int32_t e = (int32_t)((u >> 23) & 0xffu);
    uint32_t m = u & 0x7fffffu;
    if (e == 255) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u | (m >> 13) : 0u));
    int32_t eh = e - 127 + 15;
    if (eh >= 31) return (uint16_t)(sign | 0x7c00u);
    if (eh <= 0) {
        if (eh < -10) return (uint16_t)sign; /* below half the smallest subnormal: +-0 */
        m |= 0x800000u;                       /* implicit bit */
        uint32_t sh = (uint32_t)(14 - eh);    /* 14..24 */
        uint32_t r = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r); /* a carry into bit 10 gives the smallest normal, as it should */
    }
    uint32_t r = ((uint32_t)eh << 10) | (m >> 13), rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++; /* carry may reach the exponent: correct (or inf) */
    return (uint16_t)(sign | r);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, u;
    if (e == 0) {
        if (m == 0) u = sign;
        else { /* subnormal: m * 2^-24, exact in f32 */
            float f = (float)m * 5.9604644775390625e-8f;
            memcpy(&u, &f, 4);
            u |= sign;
        }
    } else if (e == 31) u = sign | 0x7f800000u | (m << 13);
    else u = sign | ((e - 15 + 127) << 23) | (m << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_f32_to_f16_n(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_f32_to_f16(x[i]);
}

int orc_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------------------------- RoPE table ---------------------------------- */

/* engine.rs:108-114: scale = 1e7f32.powf(-2/64); th = pos as f32; c[i] = th.cos(); s[i] = th.sin(); th *= scale.
 * Rust's f32 powf/cos/sin lower to the platform libm's powf/cosf/sinf, used here too. */
void orc_rope_table(int32_t pos, float tab[64]) {
    float scale = powf(1e7f, -2.0f / 64.0f);
    float th = (float)pos;
    for (int i = 0; i < 32; i++) {
        tab[i] = cosf(th);
        tab[32 + i] = sinf(th);
        th = th * scale;
    }
}

/* ---------------------------------------------------------------- append -------------------------------------- */

/* kv_src (kv.wgsl:19-23): value of dim d of one K row after NEOX RoPE on dims 0..63, pairs (i, i+32). */
static float kv_src(const float* a, int d, const float* tb) {
    if (d < 32) {
        float p1 = a[d] * tb[d];
        float p2 = a[d + 32] * tb[32 + d];
        return p1 - p2;
    }
    if (d < 64) {
        int i = d - 32;
        float p1 = a[i] * tb[32 + i];
        float p2 = a[d] * tb[i];
        return p1 + p2;
    }
    return a[d];
}

void orc_append(int fmt, void* kc, void* vc, int pos, int ntok, const float* kn, const float* v, const float* tab) {
    for (int t = 0; t < ntok; t++) {
        for (int kvh = 0; kvh < ORC_KVH; kvh++) {
            /* kv_rope2 row r = t*2 + kvh: source at r*256, table (r / flag)*64 with flag = 2, written at
             * extra + r*256 with extra = pos*512 (quad.rs:282, engine.rs:1213) */
            const float* a = kn + ((size_t)t * ORC_KVH + kvh) * ORC_D;
            const float* tb = tab + (size_t)t * 64;
            size_t o = (size_t)(pos + t) * ORC_ROW + (size_t)kvh * ORC_D;
            for (int d = 0; d < ORC_D; d++) {
                float val = kv_src(a, d, tb);
                if (fmt == 0) ((uint16_t*)kc)[o + d] = orc_f32_to_f16(val);
                else ((float*)kc)[o + d] = val;
            }
        }
        /* kv_copy / copy: 512 contiguous values of token t at (pos + t)*512 */
        size_t o = (size_t)(pos + t) * ORC_ROW;
        for (int e = 0; e < ORC_ROW; e++) {
            float val = v[(size_t)t * ORC_ROW + e];
            if (fmt == 0) ((uint16_t*)vc)[o + e] = orc_f32_to_f16(val);
            else ((float*)vc)[o + e] = val;
        }
    }
}

/* f32 fetch of element (pos, kvh, d) of a cache in either format */
static inline float kvget(int fmt, const void* c, size_t idx) {
    return fmt == 0 ? orc_f16_to_f32(((const uint16_t*)c)[idx]) : ((const float*)c)[idx];
}

/* ---------------------------------------------------------------- merge --------------------------------------- */

/* attn_fd_combine (ops.wgsl:523-538) for one (token, head): partials [m, l, acc[256]] of nbv valid blocks. */
static void combine(const float* part, int nbv, float* out) {
    float M = NEG_BIG;
    for (int b = 0; b < nbv; b++) M = fmaxf(M, part[(size_t)b * 258]);
    float tot = 0.0f;
    float acc[ORC_D];
    for (int d = 0; d < ORC_D; d++) acc[d] = 0.0f;
    for (int b = 0; b < nbv; b++) {
        const float* p = part + (size_t)b * 258;
        float e = expf(p[0] - M);
        tot += e * p[1];
        for (int d = 0; d < ORC_D; d++) acc[d] += e * p[2 + d];
    }
    for (int d = 0; d < ORC_D; d++) out[d] = acc[d] / tot;
}

/* ---------------------------------------------------------------- attn_fd ------------------------------------- */

/* attn_fd_one (ops.wgsl:333-394): one (kvh, block, token) work unit for the 8 heads of kvh. Scores in f32, exact
 * block max, w = exp(s - max) in f32, acc[h][d] = sum w * v. Writes partial [m, l, acc] per head. */
static void fd_unit(int fmt, const void* kc, const void* vc, const float* qt, int kvh, int s0, int s1, float scale,
                    float* part_h0, size_t part_stride) {
    int nb = s1 - s0;
    float* sc = (float*)malloc(sizeof(float) * 8 * (size_t)nb);
    for (int j = 0; j < nb; j++) {
        size_t kb = (size_t)(s0 + j) * ORC_ROW + (size_t)kvh * ORC_D;
        for (int h = 0; h < 8; h++) {
            const float* q = qt + (size_t)(8 * kvh + h) * ORC_D;
            float s = 0.0f;
            for (int d = 0; d < ORC_D; d++) s += q[d] * kvget(fmt, kc, kb + d);
            sc[h * nb + j] = s * scale;
        }
    }
    for (int h = 0; h < 8; h++) {
        float* p = part_h0 + (size_t)h * part_stride;
        float mx = NEG_BIG;
        for (int j = 0; j < nb; j++) mx = fmaxf(mx, sc[h * nb + j]);
        float sm = 0.0f;
        for (int j = 0; j < nb; j++) {
            float w = expf(sc[h * nb + j] - mx);
            sc[h * nb + j] = w;
            sm += w;
        }
        p[0] = mx;
        p[1] = sm;
        for (int d = 0; d < ORC_D; d++) p[2 + d] = 0.0f;
        for (int j = 0; j < nb; j++) {
            size_t vb = (size_t)(s0 + j) * ORC_ROW + (size_t)kvh * ORC_D;
            float w = sc[h * nb + j];
            for (int d = 0; d < ORC_D; d++) p[2 + d] += w * kvget(fmt, vc, vb + d);
        }
    }
    free(sc);
}

void orc_attn_fd(int fmt, const void* kc, const void* vc, const float* q, int ntok, int n, int start, float scale,
                 int bb, float* out) {
    int nbmax = (n + ntok - 1 - start + bb - 1) / bb;
    float* part = (float*)malloc(sizeof(float) * 258 * (size_t)ntok * ORC_H * (size_t)nbmax);
    int units = ntok * ORC_KVH * nbmax;
#pragma omp parallel for schedule(dynamic, 1)
    for (int u = 0; u < units; u++) {
        int t = u / (ORC_KVH * nbmax), kvh = (u / nbmax) % ORC_KVH, b = u % nbmax;
        int nt = n + t; /* token t sees [start, n + t) */
        int s0 = start + b * bb, s1 = s0 + bb < nt ? s0 + bb : nt;
        if (s0 >= nt) continue; /* block past the valid positions: not merged */
        float* p = part + (((size_t)t * ORC_H + 8 * kvh) * nbmax + b) * 258;
        fd_unit(fmt, kc, vc, q + (size_t)t * ORC_H * ORC_D, kvh, s0, s1, scale, p, (size_t)nbmax * 258);
    }
#pragma omp parallel for
    for (int r = 0; r < ntok * ORC_H; r++) {
        int t = r / ORC_H;
        int nbv = (n + t - start + bb - 1) / bb;
        combine(part + (size_t)r * nbmax * 258, nbv, out + (size_t)r * ORC_D);
    }
    free(part);
}

/* ---------------------------------------------------------------- attn_dmx ------------------------------------ */

#define DM_LAZY 8.0f

/* One (kvh, chunk) work unit of attn_dmx{r} (dmx.rs:40-114) for rows r = t*8 + head, t < ntok. */
static void dmx_unit(const uint16_t* kc, const uint16_t* vc, const float* qh /*[32][256] f16-rounded, kvh's rows*/,
                     int kvh, int chunk, int ch, int ntok, int n, float scale, float* part, int nchunk) {
    int m = 8 * ntok;
    int cs = chunk * ch;
    int lim = n + ntok - 1; /* the last token sees positions [0, lim) */
    if (cs >= lim) return;
    int nt = (lim - cs + 63) / 64;
    int ntile = ch / 64 < nt ? ch / 64 : nt;
    float mm[32], ml[32], O[32][ORC_D], S[32][64], P[32][64];
    for (int r = 0; r < m; r++) {
        mm[r] = NEG_BIG;
        ml[r] = 0.0f;
        for (int d = 0; d < ORC_D; d++) O[r][d] = 0.0f;
    }
    for (int tile = 0; tile < ntile; tile++) {
        int k0 = cs + tile * 64;
        /* S = Q K^T on f16 operands, f32 sums */
        for (int j = 0; j < 64; j++) {
            if (k0 + j >= lim) { /* past every row's window: masked below; not read (the array may end here) */
                for (int r = 0; r < m; r++) S[r][j] = 0.0f;
                continue;
            }
            size_t kb = (size_t)(k0 + j) * ORC_ROW + (size_t)kvh * ORC_D;
            float kr[ORC_D];
            for (int d = 0; d < ORC_D; d++) kr[d] = orc_f16_to_f32(kc[kb + d]);
            for (int r = 0; r < m; r++) {
                float s = 0.0f;
                for (int d = 0; d < ORC_D; d++) s += qh[r * ORC_D + d] * kr[d];
                S[r][j] = s;
            }
        }
        for (int r = 0; r < m; r++) {
            int vis = n + r / 8; /* the token of row r sees positions < vis */
            float mt = NEG_BIG;
            for (int j = 0; j < 64; j++) {
                float v = (k0 + j < vis) ? S[r][j] * scale : NEG_BIG;
                S[r][j] = v;
                mt = fmaxf(mt, v);
            }
            float mo = mm[r], mr = mo;
            if (mo < -1.0e38f || mt > mo + DM_LAZY) mr = fmaxf(mo, mt);
            float sm = 0.0f;
            for (int j = 0; j < 64; j++) {
                float v = S[r][j];
                float w = v > -1.0e38f ? expf(v - mr) : 0.0f;
                float wh = orc_f16_to_f32(orc_f32_to_f16(w));
                P[r][j] = wh;
                sm += wh;
            }
            float cf = mo > -1.0e38f ? expf(mo - mr) : 1.0f;
            mm[r] = mr;
            ml[r] = ml[r] * cf + sm;
            if (cf != 1.0f)
                for (int d = 0; d < ORC_D; d++) O[r][d] *= cf;
        }
        /* O += P V (f16 P, f16 V, f32 sums) */
        for (int j = 0; j < 64; j++) {
            if (k0 + j >= lim) continue; /* P = 0 for every row */
            size_t vb = (size_t)(k0 + j) * ORC_ROW + (size_t)kvh * ORC_D;
            float vr[ORC_D];
            for (int d = 0; d < ORC_D; d++) vr[d] = orc_f16_to_f32(vc[vb + d]);
            for (int r = 0; r < m; r++) {
                float p = P[r][j];
                if (p == 0.0f) continue;
                for (int d = 0; d < ORC_D; d++) O[r][d] += p * vr[d];
            }
        }
    }
    for (int r = 0; r < m; r++) {
        int t = r / 8, head = 8 * kvh + r % 8;
        float* p = part + (((size_t)t * ORC_H + head) * nchunk + chunk) * 258;
        p[0] = mm[r];
        p[1] = ml[r];
        for (int d = 0; d < ORC_D; d++) p[2 + d] = O[r][d];
    }
}

void orc_attn_dmx(const uint16_t* kc, const uint16_t* vc, const float* q, int ntok, int n, float scale, int ch,
                  float* out) {
    int lim = n + ntok - 1;
    int nchunk = (lim + ch - 1) / ch;
    /* q_dmx (dmx.rs:128-138): Q to f16, [kvh][row = t*8 + head][256] */
    float* qh = (float*)malloc(sizeof(float) * ORC_KVH * 32 * ORC_D);
    for (int kvh = 0; kvh < ORC_KVH; kvh++)
        for (int r = 0; r < 32; r++)
            for (int d = 0; d < ORC_D; d++) {
                int t = r / 8, head = 8 * kvh + r % 8;
                float v = t < ntok ? q[((size_t)t * ORC_H + head) * ORC_D + d] : 0.0f;
                qh[((size_t)kvh * 32 + r) * ORC_D + d] = orc_f16_to_f32(orc_f32_to_f16(v));
            }
    float* part = (float*)calloc(258 * (size_t)ntok * ORC_H * (size_t)nchunk, sizeof(float));
#pragma omp parallel for schedule(dynamic, 1)
    for (int u = 0; u < ORC_KVH * nchunk; u++) {
        int kvh = u / nchunk, c = u % nchunk;
        dmx_unit(kc, vc, qh + (size_t)kvh * 32 * ORC_D, kvh, c, ch, ntok, n, scale, part, nchunk);
    }
#pragma omp parallel for
    for (int r = 0; r < ntok * ORC_H; r++) {
        int t = r / ORC_H;
        int nbv = (n + t + ch - 1) / ch;
        combine(part + (size_t)r * nchunk * 258, nbv, out + (size_t)r * ORC_D);
    }
    free(part);
    free(qh);
}

/* ---------------------------------------------------------------- prefill ------------------------------------- */

/* One (kvh, chunk, token) unit of the online-softmax flash attention of the prefill, for the 8 heads of kvh:
 * attn_fa_mx (fa_mx.wgsl:19-115) when qk_f16 = 1 (Q and K rounded to f16 for S; f16 cache), attn_fa (ops.wgsl:540-651)
 * when qk_f16 = 0 (f32 cache, f32 math). 64-key tiles, exact running max, P in f32, l and acc rescaled by
 * cf = exp(m_old - m_new) (0 when the row had no key yet). */
static void fa_unit(int qk_f16, const void* kc, const void* vc, const float* qt /*[16][256]*/, int kvh, int cs,
                    int ce, int vis, float scale, float* part_h0, size_t part_stride) {
    int fmt = qk_f16 ? 0 : 1;
    float qr[8][ORC_D];
    for (int h = 0; h < 8; h++)
        for (int d = 0; d < ORC_D; d++) {
            float v = qt[(size_t)(8 * kvh + h) * ORC_D + d];
            qr[h][d] = qk_f16 ? orc_f16_to_f32(orc_f32_to_f16(v)) : v;
        }
    float mm[8], ml[8], acc[8][ORC_D];
    for (int h = 0; h < 8; h++) {
        mm[h] = NEG_BIG;
        ml[h] = 0.0f;
        for (int d = 0; d < ORC_D; d++) acc[h][d] = 0.0f;
    }
    for (int k0 = cs; k0 < ce; k0 += 64) {
        float S[8][64];
        for (int j = 0; j < 64; j++) {
            int key = k0 + j;
            if (key >= vis || key >= ce) {
                for (int h = 0; h < 8; h++) S[h][j] = NEG_BIG;
                continue;
            }
            size_t kb = (size_t)key * ORC_ROW + (size_t)kvh * ORC_D;
            float kr[ORC_D];
            for (int d = 0; d < ORC_D; d++) kr[d] = kvget(fmt, kc, kb + d);
            for (int h = 0; h < 8; h++) {
                float s = 0.0f;
                for (int d = 0; d < ORC_D; d++) s += qr[h][d] * kr[d];
                S[h][j] = s * scale;
            }
        }
        for (int h = 0; h < 8; h++) {
            float mo = mm[h], mx = mo;
            for (int j = 0; j < 64; j++) mx = fmaxf(mx, S[h][j]);
            float sm = 0.0f;
            for (int j = 0; j < 64; j++) {
                float v = S[h][j];
                float w = v > -1.0e38f ? expf(v - mx) : 0.0f;
                S[h][j] = w;
                sm += w;
            }
            float cf = mo > -1.0e38f ? expf(mo - mx) : 0.0f;
            mm[h] = mx;
            ml[h] = ml[h] * cf + sm;
            for (int d = 0; d < ORC_D; d++) acc[h][d] *= cf;
        }
        for (int j = 0; j < 64; j++) {
            int key = k0 + j;
            if (key >= vis || key >= ce) continue;
            size_t vb = (size_t)key * ORC_ROW + (size_t)kvh * ORC_D;
            float vr[ORC_D];
            for (int d = 0; d < ORC_D; d++) vr[d] = kvget(fmt, vc, vb + d);
            for (int h = 0; h < 8; h++) {
                float p = S[h][j];
                for (int d = 0; d < ORC_D; d++) acc[h][d] += p * vr[d];
            }
        }
    }
    for (int h = 0; h < 8; h++) {
        float* p = part_h0 + (size_t)h * part_stride;
        p[0] = mm[h];
        p[1] = ml[h];
        for (int d = 0; d < ORC_D; d++) p[2 + d] = acc[h][d];
    }
}

static void fa_common(int qk_f16, const void* kc, const void* vc, const float* q, int T, int n, int start,
                      float scale, int ch, const int* sel, int nsel, float* out) {
    if (!sel) nsel = T;
    int maxt = 0;
    for (int i = 0; i < nsel; i++) {
        int t = sel ? sel[i] : i;
        if (t > maxt) maxt = t;
    }
    int nchunk = (n + maxt - start + ch - 1) / ch;
    float* part = (float*)malloc(sizeof(float) * 258 * (size_t)nsel * ORC_H * (size_t)nchunk);
    int units = nsel * ORC_KVH * nchunk;
#pragma omp parallel for schedule(dynamic, 1)
    for (int u = 0; u < units; u++) {
        int i = u / (ORC_KVH * nchunk), kvh = (u / nchunk) % ORC_KVH, c = u % nchunk;
        int t = sel ? sel[i] : i;
        int vis = n + t; /* token t sees [start, n + t) */
        int cs = start + c * ch, ce = cs + ch;
        if (cs >= vis) continue;
        float* p = part + (((size_t)i * ORC_H + 8 * kvh) * nchunk + c) * 258;
        fa_unit(qk_f16, kc, vc, q + (size_t)t * ORC_H * ORC_D, kvh, cs, ce, vis, scale, p, (size_t)nchunk * 258);
    }
#pragma omp parallel for
    for (int r = 0; r < nsel * ORC_H; r++) {
        int i = r / ORC_H;
        int t = sel ? sel[i] : i;
        int nbv = (n + t - start + ch - 1) / ch;
        combine(part + (size_t)r * nchunk * 258, nbv, out + (size_t)r * ORC_D);
    }
    free(part);
}

void orc_attn_fa_mx(const uint16_t* kc, const uint16_t* vc, const float* q, int T, int n, int start, float scale,
                    int ch, const int* sel, int nsel, float* out) {
    fa_common(1, kc, vc, q, T, n, start, scale, ch, sel, nsel, out);
}

void orc_attn_fa_f32(const float* kc, const float* vc, const float* q, int T, int n, int start, float scale,
                     const int* sel, int nsel, float* out) {
    fa_common(0, kc, vc, q, T, n, start, scale, 2048, sel, nsel, out);
}

/* ---------------------------------------------------------------- attn_fd4 ------------------------------------ */

/* One (kvh, block of bl positions, token) unit of attn_fd4 (ops.wgsl:709-778) for the 8 heads of kvh: the block's
 * positions in tiles of 64 (F4_B); scores are sums over the 64 vec4 groups of the row of dot(q4, k4) (each dot summed
 * left to right), times scale, -3e38 for positions >= vis; per tile the exact running max mx = max(m, tile), the
 * shrink cf = exp(m - mx) (0 while m is -3e38), w = exp(s - mx) (0 for masked scores), l = l * cf + sum w,
 * acc = acc * cf + sum w * v. Partial [m, l, acc] per head. */
static void fd4_unit(int fmt, const void* kc, const void* vc, const float* qt, int kvh, int b0, int bl, int vis,
                     float scale, float* part_h0, size_t part_stride) {
    float mm[8], ml[8], acc[8][ORC_D];
    for (int h = 0; h < 8; h++) {
        mm[h] = NEG_BIG;
        ml[h] = 0.0f;
        for (int d = 0; d < ORC_D; d++) acc[h][d] = 0.0f;
    }
    for (int t0 = b0; t0 < b0 + bl && t0 < vis; t0 += 64) {
        float S[8][64];
        for (int j = 0; j < 64; j++) {
            const int key = t0 + j;
            if (key >= vis) {
                for (int h = 0; h < 8; h++) S[h][j] = NEG_BIG;
                continue;
            }
            const size_t kb = (size_t)key * ORC_ROW + (size_t)kvh * ORC_D;
            for (int h = 0; h < 8; h++) {
                const float* q = qt + (size_t)(8 * kvh + h) * ORC_D;
                float s = 0.0f;
                for (int i = 0; i < 64; i++) {
                    const float* q4 = q + 4 * i;
                    float dt = q4[0] * kvget(fmt, kc, kb + 4 * i);
                    dt += q4[1] * kvget(fmt, kc, kb + 4 * i + 1);
                    dt += q4[2] * kvget(fmt, kc, kb + 4 * i + 2);
                    dt += q4[3] * kvget(fmt, kc, kb + 4 * i + 3);
                    s += dt;
                }
                S[h][j] = s * scale;
            }
        }
        for (int h = 0; h < 8; h++) {
            float mx = mm[h];
            for (int j = 0; j < 64; j++) mx = fmaxf(mx, S[h][j]);
            const float cf = mm[h] > -1.0e38f ? expf(mm[h] - mx) : 0.0f;
            float sm = 0.0f;
            for (int j = 0; j < 64; j++) {
                const float v = S[h][j];
                const float w = v > -1.0e38f ? expf(v - mx) : 0.0f;
                S[h][j] = w;
                sm += w;
            }
            mm[h] = mx;
            ml[h] = ml[h] * cf + sm;
            for (int d = 0; d < ORC_D; d++) acc[h][d] *= cf;
        }
        for (int j = 0; j < 64 && t0 + j < vis; j++) {
            const size_t vb = (size_t)(t0 + j) * ORC_ROW + (size_t)kvh * ORC_D;
            for (int d = 0; d < ORC_D; d++) {
                const float vv = kvget(fmt, vc, vb + d);
                for (int h = 0; h < 8; h++) acc[h][d] += S[h][j] * vv;
            }
        }
    }
    for (int h = 0; h < 8; h++) {
        float* p = part_h0 + (size_t)h * part_stride;
        p[0] = mm[h];
        p[1] = ml[h];
        for (int d = 0; d < ORC_D; d++) p[2 + d] = acc[h][d];
    }
}

void orc_attn_fd4(int fmt, const void* kc, const void* vc, const float* q, int T, int n, float scale, int bl,
                  float* out) {
    const int nbmax = (n + T - 1 + bl - 1) / bl;
    float* part = (float*)malloc(sizeof(float) * 258 * (size_t)T * ORC_H * (size_t)nbmax);
    const int units = T * ORC_KVH * nbmax;
#pragma omp parallel for schedule(dynamic, 1)
    for (int u = 0; u < units; u++) {
        const int t = u / (ORC_KVH * nbmax), kvh = (u / nbmax) % ORC_KVH, b = u % nbmax;
        const int vis = n + t; /* token t sees [0, n + t) (extra = 0 in the prefill, engine.rs:920-921) */
        if (b * bl >= vis) continue; /* not written; the merge takes the valid blocks only */
        float* p = part + (((size_t)t * ORC_H + 8 * kvh) * nbmax + b) * 258;
        fd4_unit(fmt, kc, vc, q + (size_t)t * ORC_H * ORC_D, kvh, b * bl, bl, vis, scale, p, (size_t)nbmax * 258);
    }
#pragma omp parallel for
    for (int r = 0; r < T * ORC_H; r++) {
        const int t = r / ORC_H;
        const int nbv = (n + t + bl - 1) / bl; /* attn_fd_combine with flag = bl (ops.wgsl:527-528) */
        combine(part + (size_t)r * nbmax * 258, nbv, out + (size_t)r * ORC_D);
    }
    free(part);
}

/* ---------------------------------------------------------------- gate ---------------------------------------- */

void orc_gate(const float* att, const float* qf, int ntok, float* out) {
    for (int t = 0; t < ntok; t++)
        for (int i = 0; i < ORC_H * ORC_D; i++) {
            int h = i / ORC_D, d = i % ORC_D;
            float g = qf[(size_t)t * ORC_H * 512 + (size_t)h * 512 + 256 + d];
            float s = 1.0f / (1.0f + expf(-g));
            out[(size_t)t * ORC_H * ORC_D + i] = att[(size_t)t * ORC_H * ORC_D + i] * s;
        }
}

/* attn_gate16 (ops.wgsl:296-300): the same product, a[i] * sigm(b[h*512 + 256 + d]), written as f16 pairs by
 * pack2x16float (round to nearest even); the 4-token verify (quad.rs:125) and the f16-activation 2-token step
 * (engine.rs:1103) write their gated attention this way. */
void orc_gate16(const float* att, const float* qf, int ntok, uint16_t* out) {
    for (int t = 0; t < ntok; t++)
        for (int i = 0; i < ORC_H * ORC_D; i++) {
            int h = i / ORC_D, d = i % ORC_D;
            float g = qf[(size_t)t * ORC_H * 512 + (size_t)h * 512 + 256 + d];
            float s = 1.0f / (1.0f + expf(-g));
            out[(size_t)t * ORC_H * ORC_D + i] = orc_f32_to_f16(att[(size_t)t * ORC_H * ORC_D + i] * s);
        }
}

/* rmsnorm (ops.wgsl:27-57) for rows of 256 values, as the q/k norms call it (uniforms qn / kn, quad.rs:50;
 * engine.rs:965, :1182; f1 = 1, flag = 1: weight, no gate): one work-group of 256 threads per row, thread t holds
 * x[t]^2, then the shared-memory tree partial[t] += partial[t + m] for m = 128, 64, .., 1; scale = 1 / sqrt(sum / n +
 * eps) with a correctly rounded square root and division; y = ((x * scale) * 1) * w, no contraction. */
static void rmsnorm_row(const float* x, const float* w, float eps, float* y) {
    float part[256];
    for (int t = 0; t < 256; t++) part[t] = x[t] * x[t];
    for (int m = 128; m > 0; m >>= 1)
        for (int t = 0; t < m; t++) part[t] = part[t] + part[t + m];
    const float scale = 1.0f / sqrtf(part[0] / 256.0f + eps);
    for (int t = 0; t < 256; t++) y[t] = (x[t] * scale) * 1.0f * w[t];
}

void orc_rmsnorm_rows(const float* x, int rows, int step, const float* w, float eps, float* y) {
    for (int r = 0; r < rows; r++) rmsnorm_row(x + (size_t)r * step, w, eps, y + (size_t)r * 256);
}

/* The q/k producer of one block of ntok tokens (quad.rs:113-115, engine.rs:1210-1212): q rows qf[t][h][0..256)
 * (qf = [ntok][16][512], q then gate per head) RMS-normed with q_w and rotated by rope2 (ops.wgsl:275-286: dims
 * t < 32: x1*c - x2*s and x1*s + x2*c at t + 32, dims >= 64 copied) with token t's table row; k rows kb[t][kvh]
 * RMS-normed with k_w (their rotation is the append's). */
void orc_qk_norm_rope(const float* qf, const float* kb, int ntok, const float* q_w, const float* k_w, float eps,
                      const float* tab /*[ntok][64]*/, float* q_out /*[ntok][16][256]*/, float* kn_out /*[ntok][2][256]*/) {
    float y[256];
    for (int t = 0; t < ntok; t++) {
        const float* tb = tab + (size_t)t * 64;
        for (int h = 0; h < 16; h++) {
            rmsnorm_row(qf + ((size_t)t * 16 + h) * 512, q_w, eps, y);
            float* o = q_out + ((size_t)t * 16 + h) * 256;
            for (int i = 0; i < 32; i++) {
                const float x1 = y[i], x2 = y[i + 32], c = tb[i], sn = tb[32 + i];
                o[i] = x1 * c - x2 * sn;
                o[i + 32] = x1 * sn + x2 * c;
            }
            for (int d = 64; d < 256; d++) o[d] = y[d];
        }
        orc_rmsnorm_rows(kb + (size_t)t * 512, 2, 256, k_w, eps, kn_out + (size_t)t * 512);
    }
}

