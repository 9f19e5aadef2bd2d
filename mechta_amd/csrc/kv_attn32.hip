// kv_attn32.hip -- decode attention over the f32 store: 1-4 tokens (the reference's exact-f32 attn_fd applied per
// token with the drafts' causal mask, ops.wgsl:310-394, quad.rs:127-131), with the fused append. The f32 store's
// prefill is prefill_f32 (kv_prefill.hip).
//
// Work-group (block of 4 tokens, key split, kv head): 32 query rows (token * 8 + head) against the split's keys in
// tiles of 32 keys, by 4 waves.
//
// f32 products on the f16 matrix units: each f32 operand x is split into hi = f16(x) and lo = f16(x - hi), and a
// product a.b is taken as hi(a)hi(b) + hi(a)lo(b) + lo(a)hi(b) (three v_mfma_f32_32x32x16_f16, f32 accumulation; the
// dropped lo.lo term is below 2^-22 of |a||b|). The f16 matrix units run 32x32x16 in the time the f32 ones take for
// 32x32x2, so the three passes cost 3/8 of one f32 pass, and the path keeps f32-level accuracy (within 1e-5 of the
// exact-f32 reference). Per tile, wave w of a group computes
//   S^T[32 keys][32 rows] over dims 64w .. 64w+63    4 dim steps x 3 passes; A = K split from its HBM loads, B = Q
//                                                     (split once into LDS)
//   the four partial S^T summed through LDS ((w0 + w1) + (w2 + w3), the same order in every wave)
//   exact-max online softmax of the 32 rows (each wave redundantly: 16 scores per lane)
//   O[32 rows][dims 64w .. 64w+63] += P . V           2 key steps x 2 dim blocks x 3 passes; A = P split from the
//                                                     S^T registers, B = V split from its HBM loads
// The 32x32 accumulator layout gives lane l (half s = l / 32) row l % 32 and keys 8a + 4s + b (register 4a + b). A
// 16-key step k of P.V takes, in lane half s, the keys 16k + 4s + b and 16k + 8 + 4s + b (b < 4): the step's keys
// are summed in any order as long as P and V agree on it, so P never leaves the registers, and with V stored
// [pos/4][d][pos%4] each four keys of a dim are one 16-byte load. K is stored [pos/32][d/4][pos%32][4]: a lane's
// 16-byte K load is 4 dims of key l % 32. Tiles are double-buffered in registers: the loads of tile j + 1 fly while
// tile j computes.
#include "mkv_device.h"

namespace mkv {
namespace {

constexpr int TILE = 32;                       // keys per tile: one K block, eight V groups
constexpr unsigned TILE_BYTES = TILE * HD * 4;  // 32 KB of each plane
constexpr int QPAD = HD + 8;                   // LDS row of Q's halves: 16-byte reads of 32 rows conflict-free

// voff: the lane's offset (fixed for the kernel), soff: the wave-uniform tile offset in the scalar operand (no vector
// instruction per load for the tile base)
__device__ inline f32x4 bload4f(rsrc_t r, unsigned voff, unsigned soff) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, LOAD_NT));
}

#ifndef ATTN32_NWV
#define ATTN32_NWV 4
#endif
constexpr int NWV = ATTN32_NWV;   // waves per work-group, each over DPW of the 256 dims
constexpr int DPW = HD / NWV;     // 64 (4 waves) or 32 (8 waves)
constexpr int NC = DPW / 32;      // 32-dim blocks of P.V per wave
constexpr int NTH = 64 * NWV;     // threads per work-group
struct Tile {
    f32x4 k[DPW / 8];  // K: dims DPW w + 16k + 8s + 4e .. +3 of key l % 32 (index 2k + e)
    f32x4 v[4 * NC];   // V: keys 16k + 8e + 4s .. +3 of dim DPW w + 32c + l % 32 (index 2 NC k + 2c + e)
};

// Two tiles in registers, one loading while the other computes (deeper prefetch measured slower from HBM: 3 tiles 2 us
// and 4 tiles 5 us more per 16K-position decode)
__global__ void __launch_bounds__(NTH, NWV == 4 ? 2 : 1) attn_f32(const float* __restrict__ kplane, const float* __restrict__ vplane,
                                                size_t plane_elems, const float* __restrict__ q, int T, int n,
                                                int start, float scale2, int span, int nch, int c0, int nrb, int rpk,
                                                float* __restrict__ part, const float* __restrict__ akn,
                                                const float* __restrict__ av, const float* __restrict__ atab, int apos,
                                                int antok) {
    // XCD-aware order: consecutive work-groups go round robin to the 8 XCDs, so work item W = (L % 8) (G / 8) + L / 8
    // puts the token blocks that stream the same keys on one XCD's L2
    const int G = gridDim.x, L = blockIdx.x;
    const int W = G % NXCD == 0 ? (L % NXCD) * (G / NXCD) + L / NXCD : L;
    const int ncg = nch - c0;
    const int rb = W % nrb, c = c0 + (W / nrb) % ncg, kvh = W / nrb / ncg;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, s = lane >> 5, r32 = lane & 31;
    const int t0 = 4 * rb, nt = min(4, T - t0);
    const int kend = n + T - 1;  // keys of the whole call
    // span > 0: work-group c takes the contiguous split [chunk_lo(c), chunk_lo(c + 1)) (prefill: the token blocks of
    // a split share its keys through one L2). span == 0 (decode): the 32-key tiles from the window start on are dealt
    // round robin, tile c + j * nch to work-group c, so at any moment the work-groups stream neighbouring tiles.
    int lo, hi, ntile, tstep;  // tile j of this work-group starts at key lo + j * tstep * TILE; keys < hi are its
    if (span > 0) {
        const int cs = chunk_lo(c, span, nch), ce = c + 1 < nch ? chunk_lo(c + 1, span, nch) : kend;
        lo = max(cs, start / TILE * TILE);
        hi = min(ce, n + t0 + nt - 1);  // the block's last key + 1
        ntile = hi > lo ? (hi - lo + TILE - 1) / TILE : 0;
        tstep = 1;
    } else {
        const int lo0 = start / TILE * TILE;
        hi = n + t0 + nt - 1;
        const int nt_all = (hi - lo0 + TILE - 1) / TILE;
        lo = lo0 + c * TILE;
        ntile = c < nt_all ? (nt_all - c + nch - 1) / nch : 0;
        tstep = nch;
    }

    // tile j of this split starts at key lo + 32j, at the same byte offset j * 32 KB in both planes; loads of tile
    // ntile (the prefetch after the last) lie past the resources and return zeros without a memory access
    const unsigned rbytes = ntile > 0 ? (unsigned)((ntile - 1) * tstep + 1) * TILE_BYTES : 0u;
    const rsrc_t kr = plane_rsrc(kplane + (size_t)kvh * plane_elems + (size_t)lo * HD, rbytes);
    const rsrc_t vr = plane_rsrc(vplane + (size_t)kvh * plane_elems + (size_t)lo * HD, rbytes);
    const unsigned kofs = (((DPW / 4) * w + 2 * s) * TILE + r32) * 16;  // + (4k + e) * 512 B: dims DPW w + 16k + 8s + 4e
    const unsigned vofs = (s * HD + DPW * w + r32) * 16;  // + (4k + 2e) * 4 KB + c * 32 dims * 16 B
    auto load = [&](Tile& X, int j) {
        const unsigned base = __builtin_amdgcn_readfirstlane((unsigned)(j * tstep) * TILE_BYTES);
#pragma unroll
        for (int i = 0; i < DPW / 8; i++) X.k[i] = bload4f(kr, kofs + ((i >> 1) * 4 + (i & 1)) * (TILE * 16), base);
#pragma unroll
        for (int i = 0; i < 4 * NC; i++)
            X.v[i] = bload4f(vr, vofs + ((i / (2 * NC)) * 4 + 2 * (i & 1)) * (HD * 16) + ((i >> 1) % NC) * (32 * 16),
                             base);
    };

    // Fused append (decode only: mkv_append_decode on the f32 store). The new rows [apos, apos + antok) lie in the
    // last one or two tiles; the work-group holding a tile computes its new rows (the same arithmetic as
    // append_kernel) into LDS, patches them into that tile's K and V registers, and stores them to the planes after
    // its loop: no load waits for the stores, and no other work-group reads those positions in this launch.
    __shared__ __attribute__((aligned(16))) float newk[4][HD], newv[4][HD];
    __shared__ __attribute__((aligned(16))) _Float16 qh[ROWS][QPAD], ql[ROWS][QPAD];  // Q split: hi, lo
    __shared__ f32x4 sx[2][NWV][4][64];  // partial S^T of the loop: [tile parity][wave][register quad][lane]
    // the append's inputs (K normed rows, V rows, table rows) before the loop, in the S^T exchange's second buffer: a
    // buffer of their own would take the work-group's LDS past half of the CU's, and the compiler, counting on one
    // work-group per CU, would then spend registers more freely (AGPR copies in the loop: 0.85 us per cfg5 verify)
    float* const ain = (float*)&sx[1][0][0][0];
    static_assert(sizeof(sx[1]) >= (8 * HD + 4 * 64) * sizeof(float), "the append's inputs fit the second buffer");
    int apf = 0, apl = 0;  // this work-group's new rows [apf, apl)
    if (antok > 0) {
        const int lo0 = start / TILE * TILE;
        for (int p = apos; p < apos + antok; p++)
            if (((p - lo0) / TILE) % nch == c) {
                apf = apl == 0 ? p : apf;
                apl = p + 1;
            }
    }
    const int nr = apl - apf;

    if (nr > 0) {
        // the append's inputs by direct loads into LDS, issued before Q's and the tiles': they complete in order, so
        // the Q split's wait (below) covers them and not the tiles
        const int ta = apf - apos;
#pragma unroll
        for (int k = 0; k < (2 * 4 + NWV) / NWV; k++) {  // 1 KB per direct load: K rows, V rows, then the table rows
            const int i = w + NWV * k;
            if (i < 2 * nr + 1) {
                const float* src = i < nr       ? akn + ((size_t)(ta + i) * KVH + kvh) * HD
                                   : i < 2 * nr ? av + (size_t)(ta + i - nr) * (KVH * HD) + kvh * HD
                                                : atab + (size_t)ta * 64;
                const float* dst = ain + (i < nr ? i : i < 2 * nr ? 4 + i - nr : 8) * HD;
                if (i < 2 * nr || lane < 16 * nr) dma16s(src, lane * 16, (unsigned)(uintptr_t)(lds_void*)dst);
            }
        }
    }

    // Q's loads, then the first two tiles': loads complete in order, so the Q split below waits for Q only, and the
    // tiles fly while Q is split into LDS and the fused append's rows are computed
    constexpr int QI = ROWS * HD / 8 / NTH;  // 8-dim pieces of Q per thread
    f32x4 xq[QI][2];
#pragma unroll
    for (int k = 0; k < QI; k++) {
        const int i = tid + NTH * k, row = i / (HD / 8), d8 = (i % (HD / 8)) * 8, t = t0 + (row >> 3);
        const float* qr = q + ((size_t)min(t, T - 1) * QH + kvh * GQA + (row & 7)) * HD + d8;
        xq[k][0] = *(const f32x4*)qr;
        xq[k][1] = *(const f32x4*)(qr + 4);
    }
    // every Q load issued before the tiles' (a Q load the scheduler sank below them made the Q split wait for both
    // tiles: 1.4 us more per launch)
    __builtin_amdgcn_sched_barrier(0);
    Tile X[2];
    load(X[0], 0);
    load(X[1], 1);

    __shared__ __attribute__((aligned(16))) float cfw[NWV][ROWS];  // each wave's rescale factors
#pragma unroll
    for (int k = 0; k < QI; k++) {
        const int i = tid + NTH * k, row = i / (HD / 8), d8 = (i % (HD / 8)) * 8, t = t0 + (row >> 3);
        const f32x4 x0 = t < T ? xq[k][0] : f32x4{}, x1 = t < T ? xq[k][1] : f32x4{};
        half8 hi, lo;
        split8(x0, x1, hi, lo);
        *(half8*)&qh[row][d8] = hi;
        *(half8*)&ql[row][d8] = lo;
    }
    __syncthreads();
    if (nr > 0) {  // every wave's direct loads have landed: each waited for its own Q, loaded after them
        for (int i = tid; i < nr * HD; i += NTH) {
            const int r = i / HD, d = i % HD;
            newk[r][d] = rope_dim(ain + r * HD, ain + 8 * HD + r * 64, d);
            newv[r][d] = ain[(4 + r) * HD + d];
        }
        __syncthreads();
    }

    const int vis = n + t0 + (r32 >> 3);  // lane's row sees keys < vis (and of this split, < hi)
    float m_run = NEG_INF, l_run = 0.f;
    f32x16 O[NC];
#pragma unroll
    for (int cc = 0; cc < NC; cc++) O[cc] = f32x16{};
    auto step = [&](Tile& X, int j) {
        const int k0 = lo + j * tstep * TILE;
        if (k0 < apl && k0 + TILE > apf) {  // the tile holds new rows: their K and V from LDS
            const int key = k0 + r32;
            if (key >= apf && key < apl) {
#pragma unroll
                for (int i = 0; i < DPW / 8; i++)
                    X.k[i] = *(const f32x4*)&newk[key - apf][DPW * w + 16 * (i >> 1) + 8 * s + 4 * (i & 1)];
            }
#pragma unroll
            for (int i = 0; i < 4 * NC; i++)
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const int kv = k0 + 16 * (i / (2 * NC)) + 8 * (i & 1) + 4 * s + b;
                    if (kv >= apf && kv < apl) X.v[i][b] = newv[kv - apf][DPW * w + 32 * ((i >> 1) % NC) + r32];
                }
        }
        f32x16 S = f32x16{};
#pragma unroll
        for (int k = 0; k < DPW / 16; k++) {
            half8 kh, kl;
            split8(X.k[2 * k], X.k[2 * k + 1], kh, kl);
            const half8 bh = *(const half8*)&qh[r32][DPW * w + 16 * k + 8 * s];
            const half8 bl = *(const half8*)&ql[r32][DPW * w + 16 * k + 8 * s];
            S = mfma3(kh, kl, bh, bl, S);
        }
        float sv[16];
        f32x4(&sg)[NWV][4][64] = sx[j & 1];
#pragma unroll
        for (int a = 0; a < 4; a++) sg[w][a][lane] = f32x4{S[4 * a], S[4 * a + 1], S[4 * a + 2], S[4 * a + 3]};
        lds_barrier();  // parity buffers: a group's round i + 2 writes pb again only after every wave passed round i + 1
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const f32x4 p0 = sg[0][a][lane], p1 = sg[1][a][lane];
            const f32x4 p2 = sg[2][a][lane], p3 = sg[3][a][lane];
            if constexpr (NWV == 4) {
#pragma unroll
                for (int b = 0; b < 4; b++) sv[4 * a + b] = (p0[b] + p1[b]) + (p2[b] + p3[b]);
            } else {
                const f32x4 p4 = sg[4][a][lane], p5 = sg[5][a][lane];
                const f32x4 p6 = sg[6][a][lane], p7 = sg[7][a][lane];
#pragma unroll
                for (int b = 0; b < 4; b++)
                    sv[4 * a + b] = ((p0[b] + p1[b]) + (p2[b] + p3[b])) + ((p4[b] + p5[b]) + (p6[b] + p7[b]));
            }
        }
        // exact-max online softmax in log2 units on the raw scores (scale2 > 0: the max of the scaled scores is the
        // scaled max, and the exponent is one FMA); masked scores are -inf. A tile that lies inside every row's window
        // (the common case) takes no mask.
        if (!(k0 >= start && k0 + TILE <= n + t0 && k0 + TILE <= hi)) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int key = k0 + 8 * (i >> 2) + 4 * s + (i & 3);
                sv[i] = (key >= start && key < vis && key < hi) ? sv[i] : NEG_INF;
            }
        }
        // scores here are never NaN (keys of stale rows are masked above): single-instruction maxima
        float mt = vmax(sv[0], sv[1]);
#pragma unroll
        for (int i = 2; i < 16; i += 2) mt = vmax3(mt, sv[i], sv[i + 1]);
        mt = max_xor32(mt) * scale2;
        const float mn = fmaxf(m_run, mt);
        const float base = mn == NEG_INF ? 0.f : mn;
        const float cf = m_run == NEG_INF ? 0.f : fast_exp2(m_run - mn);
        float ls = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            sv[i] = fast_exp2(__builtin_fmaf(sv[i], scale2, -base));
            ls += sv[i];
        }
        ls = add_xor32(ls);
        l_run = l_run * cf + ls;
        m_run = mn;
        // rescale O: register i of this lane holds row 8(i/4) + 4s + i%4; the rows' factors pass through this wave's
        // LDS row (four 16-byte reads at constant offsets)
        if (__builtin_amdgcn_ballot_w64(cf != 1.f)) {
            if (s == 0) cfw[w][r32] = cf;
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const f32x4 f = *(const f32x4*)&cfw[w][8 * a + 4 * s];
#pragma unroll
                for (int b = 0; b < 4; b++)
#pragma unroll
                    for (int cc = 0; cc < NC; cc++) O[cc][4 * a + b] *= f[b];
            }
            __builtin_amdgcn_wave_barrier();
        }
        // keys past the block's last (unwritten or stale rows) have P = 0 and must not bring NaN in through V
        if (k0 + TILE > hi) {
#pragma unroll
            for (int i = 0; i < 4 * NC; i++)
#pragma unroll
                for (int b = 0; b < 4; b++)
                    if (k0 + 16 * (i / (2 * NC)) + 8 * (i & 1) + 4 * s + b >= hi) X.v[i][b] = 0.f;
        }
#pragma unroll
        for (int k = 0; k < 2; k++) {
            half8 ph, pl;  // P of keys 16k + 4s + b and 16k + 8 + 4s + b: registers 8k + b and 8k + 4 + b
            split8(f32x4{sv[8 * k], sv[8 * k + 1], sv[8 * k + 2], sv[8 * k + 3]},
                   f32x4{sv[8 * k + 4], sv[8 * k + 5], sv[8 * k + 6], sv[8 * k + 7]}, ph, pl);
#pragma unroll
            for (int cc = 0; cc < NC; cc++) {
                half8 vh, vl;
                split8(X.v[2 * NC * k + 2 * cc], X.v[2 * NC * k + 2 * cc + 1], vh, vl);
                O[cc] = mfma3(ph, pl, vh, vl, O[cc]);
            }
        }
    };

    // two tiles in flight from the start: step(j) computes tile j while tile j + 1 loads; its buffer then takes the
    // loads of tile j + 2
    const int rounds = ntile;
    for (int i = 0; i < rounds; i += 2) {
        step(X[0], i);
        load(X[0], i + 2);
        if (i + 1 >= rounds) break;
        step(X[1], i + 1);
        load(X[1], i + 3);
    }

    // the fused append's rows into the planes, for the launches that follow
    if (apl > apf) {
        float* Kp = (float*)kplane + (size_t)kvh * plane_elems;
        float* Vp = (float*)vplane + (size_t)kvh * plane_elems;
        for (int i = tid; i < (apl - apf) * HD; i += NTH) {
            const int r = i / HD, d = i % HD;
            Kp[k_off32(apf + r, d)] = newk[r][d];
            Vp[v_off32(apf + r, d)] = newv[r][d];
        }
    }

    // partials of the rows of present tokens: [kvh][row < rpk][chunk < nch][PART], row = token * 8 + head
    const size_t rbase = (size_t)kvh * rpk + (size_t)t0 * GQA;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int row = 8 * (i >> 2) + 4 * s + (i & 3);
        if (t0 + (row >> 3) < T) {
            float* p = part + ((rbase + row) * nch + c) * PART + PACC + DPW * w + r32;
#pragma unroll
            for (int cc = 0; cc < NC; cc++) p[32 * cc] = O[cc][i];
        }
    }
    if (w == 0 && s == 0 && t0 + (r32 >> 3) < T) {
        float* p = part + ((rbase + r32) * nch + c) * PART;
        p[0] = m_run;
        p[1] = l_run;
    }
}

}  // namespace

Attn32Plan attn32_plan(int T, int n, int start) {
    // the window's tiles dealt round robin, four per work-group, to at most 248 work-groups per kv head (registers
    // held to 256 per lane, so two work-groups share a CU past 256 of them): at 16,384 positions (128 per kv head) the
    // core takes 21.3-21.5 us, with two tiles per work-group (248) 24.7 us; per cfg5 verify three or five tiles per
    // work-group measured 30.0 and 27.0 us against 24.5, at most 108 work-groups 24.9 us. Every work-group holds keys
    // of every row, so the merge reads all (span 0)
    const int kend = n + T - 1;
    int nch = (kend - start / TILE * TILE) / 128;
    nch = nch > 248 ? 248 : nch < 1 ? 1 : nch;
    return Attn32Plan{0, nch, 0, (T + 3) / 4};
}

hipError_t launch_attn_f32(const Geom& g, const void* base, int layer, const float* q, int T, int n, int start,
                           float scale, const Attn32Plan& p, int rpk, float* part, const FusedAppend& fa,
                           const Launch& L) {
    if (fa.ntok > 0 && (p.span != 0 || fa.ntok > 4)) return hipErrorInvalidValue;  // fused append: decode plans only
    if (g.fmt != 1) return hipErrorNotSupported;
    const char* b = (const char*)base;
    const float* kp = (const float*)(b + g.plane(layer, 0, 0) * g.plane_bytes());
    const float* vp = (const float*)(b + g.plane(layer, 1, 0) * g.plane_bytes());
    if (T > 4) return hipErrorInvalidValue;  // decode only: prefill_f32 serves blocks
    dim3 grid(p.nrb * (p.nch - p.c0) * KVH);
    return launch(attn_f32, grid, dim3(NTH), L, kp, vp, g.plane_elems, q, T, n, start, scale * LOG2E, p.span,
                  p.nch, p.c0, p.nrb, rpk, part, fa.kn, fa.v, fa.tab, fa.pos, fa.ntok);
}

}  // namespace mkv
