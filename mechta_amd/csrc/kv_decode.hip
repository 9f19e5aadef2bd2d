// kv_decode.hip -- split-K flash decode for 1..4 query tokens (GQA 8:1) and the merge of the partials.
//
// Replaces attn_fd (ops.wgsl:310-394), q_dmx + attn_dmx2 (dmx.rs:19-138) and attn_fd_combine (ops.wgsl:523-538).
//
// f16 store (decode_f16): the keys are 64-position stages dealt round robin to the work-groups of a kv head (plan in
// decode_plan). The 8 query heads of the kv head times the ntok tokens are 32 query rows (row = t*8 + head, rows of
// absent tokens are zero). Per stage the 8 waves compute
//   S[64 keys][32 rows], each wave 16 keys x 128 dims   v_mfma_f32_16x16x32_f16, A = K from the blocked K plane
//   online softmax of the 32 rows, lazy reference max (moves when first or when the tile max exceeds it by > 8,
//   as attn_dmx, dmx.rs:72-74), P rounded to f16, l += f32(P)
//   O[32 rows][32 dims per wave] += P . V      v_mfma_f32_32x32x16_f16, B = V straight from the grouped V plane
// in a software pipeline with one LDS barrier per stage: K is loaded two stages ahead (for the S MFMAs, which run
// one stage ahead of the softmax) and V one stage ahead, about one stage of bytes in flight (from HBM that streams
// faster than two or three). Each work-group writes one partial [m, l, 0, 0, acc[256]] per row.
//
// The f32 store has its own kernel (kv_attn32.hip) and shares the merges below.
//
// decode_combine: one work-group per (token, head, 64 dims): o = sum_c 2^(m_c - M) acc_c / sum_c 2^(m_c - M) l_c
// over the partials holding a visible key, then the optional sigmoid output gate (attn_gate, ops.wgsl:171-177).
// Partials keep m in log2 units (scores are pre-multiplied by scale * log2 e).
#include <type_traits>

#include "mkv_device.h"

namespace mkv {
namespace {

constexpr int KPS = KPS_F16;                   // keys per stage of the decode ring
#ifndef MKV_DEC_WG
#define MKV_DEC_WG 108
#endif
// most work-groups per kv head in a decode: 2 x 108 of the 256 CUs. Measured per 4-token step (fused append, decode,
// merge; 10 layers rotated) against 124, the earlier choice, at 8,192 / 32,768 / 65,536 / 131,072 / 200,000
// positions: 14.3 / 21.2 / 29.3 / 47.5 / 66.9 us against 14.9 / 21.5 / 29.7 / 49.7 / 69.6 us. The rate is not
// monotone in the count: 100, 112 and 120 measured 0.3-0.9 us slower than 124 at 65,536 positions, 104 and 116 about
// as fast as 108 there.
constexpr int DEC_WG = MKV_DEC_WG;
constexpr int SMALL_WG = 124;                  // small prefill blocks: most work-groups per kv head and block column
constexpr int PS_STRIDE = KPS + 8;             // halves per P row in LDS (conflict-free 16-byte reads)
constexpr int QS_STRIDE = HD + 8;              // halves per Q row in LDS
constexpr int NEWMAX = 4;                      // appended rows per call
constexpr int MERGE_FEW = 16;  // chunks of the one-lane-per-dim merge
constexpr int MERGE_JMAX = 16;  // chunks per merge lane: 16 lanes x 16 >= the at most 248 splits of a decode plan

// One stage of this wave's registers: K operands (16 keys x 128 dims) and V operands (64 keys x 32 dims).
struct StageRegs {
    half8 k[4];
    half8 v[4];
};

// Stage operands in four register sets: K two stages ahead and V one stage ahead, two sets each (three or four
// sets of whole stages, two or three stages in flight, measured slower).
// EXACT = false: the reference's attn_dmx arithmetic (Q and P rounded to f16, f32 sums), for its 2- and 4-token
// steps. EXACT = true: attn_fd's f32-class arithmetic, for one token and for windows (start > 0): Q and P are split
// into f16 hi + lo and each product with the (exact f16) K or V takes two MFMA passes; the row sums add the f32 P.
template <bool EXACT>
__global__ void __launch_bounds__(512) decode_f16(_Float16* __restrict__ kplane, _Float16* __restrict__ vplane,
                                                  size_t plane_elems, const float* __restrict__ q, int ntok, int n,
                                                  int start, float scale2, int s0, int nu,
                                                  float* __restrict__ part, const float* __restrict__ akn,
                                                  const float* __restrict__ av, const float* __restrict__ atab,
                                                  int apos, int antok, int rpk, int cols) {
    // cols == 0: grid (splits, kv heads, token blocks). cols > 0 (small prefill blocks): a 1D grid of
    // splits x kv heads x cols, ordered XCD-aware with the token blocks fastest: the dispatcher deals consecutive
    // work-groups round robin to the 8 XCDs, so W = (L % 8) (G / 8) + L / 8 puts the cols work-groups that stream the
    // same stage on one XCD, where all but the first find it in L2
    int kvh = blockIdx.y, c = blockIdx.x, nch = gridDim.x, zb = blockIdx.z;
    if (cols > 0) {
        const int G = gridDim.x, L = blockIdx.x;
        const int W = G % NXCD == 0 ? (L % NXCD) * (G / NXCD) + L / NXCD : L;
        nch = G / (KVH * cols);
        zb = W % cols;
        c = (W / cols) % nch;
        kvh = W / (cols * nch);
    }
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int h = lane >> 5, r = lane & 31, l16 = lane & 15, g4 = lane >> 4;
    // the call's keys end where its last token's do; blockIdx.z = block of 4 tokens (a small prefill block runs one
    // per work-group column, with the same stages), whose token 0 sees [start, nb)
    const int kend = n + ntok - 1;
    const int nb = n + 4 * zb, ntb = min(4, ntok - 4 * zb);
    q += (size_t)4 * zb * QH * HD;
    // Stages are dealt so that the partial round comes first: with R = nu / nch and r = nu % nch, stage u >= r goes
    // to work-group (u - r) % nch, so every work-group takes R of them and the last stage (the one holding appended
    // rows) goes to work-group nch - 1. The first r stages are the partial round: when 2r <= nch they are split into
    // 2r half stages of 32 positions for work-groups 0 .. 2r - 1 (the busiest work-group then has R + 1/2 stages),
    // else stage u < r goes to work-group u.
    const int rr = nu % nch;
    const bool halves = 2 * rr <= nch;
    const int ex = c < (halves ? 2 * rr : rr);  // this work-group's stage 0 is from the partial round
    auto kbase = [&](int j) {
        return ex && j == 0 ? s0 + c * (halves ? KPS / 2 : KPS) : s0 + (rr + c + (j - ex) * nch) * KPS;
    };
    auto klen = [&](int j) { return ex && j == 0 && halves ? KPS / 2 : KPS; };
    auto owner = [&](int u) { return (u - rr) % nch; };  // of a stage u >= r (every stage that can hold new rows)
    _Float16* K = kplane + (size_t)kvh * plane_elems;
    _Float16* V = vplane + (size_t)kvh * plane_elems;

    // double-buffered by stage parity: partial S of the two dim halves [row][key], P [row][key], rescale factors
    __shared__ __attribute__((aligned(16))) float ss[2][2][ROWS][KPS + 4];
    __shared__ __attribute__((aligned(16))) _Float16 ps[2][ROWS][PS_STRIDE];
    __shared__ __attribute__((aligned(16))) float cfs[2][ROWS];
    __shared__ __attribute__((aligned(16))) _Float16 qs[ROWS][QS_STRIDE];
    __shared__ __attribute__((aligned(16))) _Float16 qsl[EXACT ? ROWS : 1][QS_STRIDE];      // EXACT: Q's lo part
    __shared__ __attribute__((aligned(16))) _Float16 psl[EXACT ? 2 : 1][ROWS][PS_STRIDE];  // EXACT: P's lo part
    // fused append: the new rows' inputs (K normed, V, RoPE table) and their f16 store values
    __shared__ __attribute__((aligned(16))) float ain[2 * NEWMAX * HD + NEWMAX * 64];
    __shared__ __attribute__((aligned(16))) _Float16 newk[NEWMAX][HD];
    __shared__ __attribute__((aligned(16))) _Float16 newv[NEWMAX][HD];

    // Roles of wave w in a 64-key stage:
    //   S: keys 16kq .. 16kq + 15 (kq = w % 4) times dims 128dh .. 128dh + 127 (dh = w / 4), both 16-row halves,
    //      v_mfma_f32_16x16x32_f16 with A = K (lane: key 16kq + lane%16, 8 dims at 32s + 8(lane/16)), B = Q^T;
    //      the two dim halves' partial S meet in LDS;
    //   P.V: dims 32w .. 32w + 31 of all 32 rows, v_mfma_f32_32x32x16_f16, B = V (lane: dim 32w + lane%32,
    //      8 keys 16s2 + 8(lane/32) .. of group 2s2 + lane/32).
    const int kq = w & 3, dh = w >> 2;
    const int nst = nu / nch + ex;
    const int kkey = 16 * kq + l16;  // S-role key inside the stage
    // Buffer loads through a resource that starts at the stage's first key and ends at the keys' end (rounded up to
    // the 32-key K block and the 8-key V group): loads past the keys, and every load of a stage past this
    // work-group's last, are out of range and move no bytes. The per-lane offsets inside a stage are loop constants.
    const int ceK = (kend + KBLK - 1) / KBLK * KBLK, ceV = (kend + VGRP - 1) / VGRP * VGRP;
    const unsigned kofs = (unsigned)(((kkey / KBLK) * (KBLK * HD) + (kkey % KBLK) * 8 + (16 * dh + g4) * (KBLK * 8)) * 2);
    const unsigned vofs = (unsigned)((h * (VGRP * HD) + (32 * w + r) * VGRP) * 2);
    auto load_k = [&](int j, StageRegs& R) {
        const int k0 = kbase(j);  // a multiple of 64: the stage starts a K block and a V group
        const rsrc_t kr = plane_rsrc(K + (size_t)k0 * HD, (unsigned)(max(min(ceK - k0, klen(j)), 0) * (HD * 2)));
#pragma unroll
        for (int s = 0; s < 4; s++) R.k[s] = bload16(kr, kofs + s * (4 * KBLK * 8 * 2));
    };
    auto load_v = [&](int j, StageRegs& R) {
        const int k0 = kbase(j);
        const rsrc_t vr = plane_rsrc(V + (size_t)k0 * HD, (unsigned)(max(min(ceV - k0, klen(j)), 0) * (HD * 2)));
#pragma unroll
        for (int s2 = 0; s2 < 4; s2++) R.v[s2] = bload16(vr, vofs + s2 * (2 * VGRP * HD * 2));
    };
    // Fused append (mkv_append_decode). The new rows [apf, apl) of the stages this work-group owns (at most two
    // stages hold new rows) are computed into LDS (the same arithmetic as append_kernel) and patched into the K and V
    // registers of the stage that holds them, so no load waits for their stores; they are stored to the planes
    // after the loop, for the launches that follow. Their inputs come into LDS by direct loads issued before Q's and
    // the stages', and a wait for all but those later loads makes them available while the stages stream.
    const int ua = antok > 0 ? (apos - s0) / KPS : 0, ub = antok > 0 ? (apos + antok - 1 - s0) / KPS : -1;
    int apf = 0, apl = 0;
    for (int u = ua; u <= ub; u++)
        if (owner(u) == c) {
            const int lo = max(apos, s0 + u * KPS), hi = min(apos + antok, s0 + (u + 1) * KPS);
            apf = apl == 0 ? lo : apf;
            apl = hi;
        }
    const int nr = apl - apf;  // 0 .. 4 new rows here, contiguous
    float* const aink = ain;
    float* const ainv = ain + NEWMAX * HD;
    float* const aint = ain + 2 * NEWMAX * HD;
    if (nr > 0) {
        const int t0 = apf - apos;
        for (int i = w; i < 2 * nr + 1; i += 8) {  // 1 KB per direct load: K rows, V rows, then the table rows
            if (i < nr)
                dma16(akn + ((size_t)(t0 + i) * KVH + kvh) * HD + 4 * lane, aink + i * HD);
            else if (i < 2 * nr)
                dma16(av + (size_t)(t0 + i - nr) * (KVH * HD) + kvh * HD + 4 * lane, ainv + (i - nr) * HD);
            else if (lane < 16 * nr)
                dma16(atab + (size_t)t0 * 64 + 4 * lane, aint);
        }
    }
    float4 xq[2][2];  // Q loads before the stages': loads complete in order, so the first stage's wait covers them
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int idx = tid + 512 * i, row = idx >> 5, d8 = (idx & 31) * 8, tq = row >> 3;
        const float* qr = q + ((size_t)min(tq, ntb - 1) * QH + kvh * GQA + (row & 7)) * HD + d8;
        xq[i][0] = *(const float4*)qr;
        xq[i][1] = *(const float4*)(qr + 4);
    }
    // three stages in flight from the start; loads of stages past this work-group's last are out of range and move
    // no bytes, so no load is behind a branch (a branch around loads makes the compiler's wait counts pessimistic)
    StageRegs R0, R1, R2, R3;  // staggered streams: K two stages ahead, V one (R0/R1 hold K, R2/R3 hold V)
    load_k(0, R0);
    load_k(1, R1);
    load_v(0, R2);
    if (nr > 0) {
        // the direct loads precede the 4 Q loads and the 12 stage loads; then every wave's LDS data is in
        asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
        for (int it = tid; it < nr * HD; it += 512) {
            const int i = it / HD, d = it % HD;
            newk[i][d] = __builtin_bit_cast(_Float16, f2h(rope_dim(aink + i * HD, aint + i * 64, d)));
            newv[i][d] = __builtin_bit_cast(_Float16, f2h(ainv[i * HD + d]));
        }
    }

    // Q rounded to f16 (as q_dmx) into LDS, [row][dim]; rows of absent tokens are zero
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int idx = tid + 512 * i, row = idx >> 5, d8 = (idx & 31) * 8, tq = row >> 3;
        float4 x0 = xq[i][0], x1 = xq[i][1];
        if (tq >= ntb) x0 = x1 = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (EXACT) {
            half8 hi, lo;
            split8(f32x4{x0.x, x0.y, x0.z, x0.w}, f32x4{x1.x, x1.y, x1.z, x1.w}, hi, lo);
            *(half8*)&qs[row][d8] = hi;
            *(half8*)&qsl[row][d8] = lo;
        } else {
            *(half8*)&qs[row][d8] = half8{(_Float16)x0.x, (_Float16)x0.y, (_Float16)x0.z, (_Float16)x0.w,
                                          (_Float16)x1.x, (_Float16)x1.y, (_Float16)x1.z, (_Float16)x1.w};
        }
    }
    lds_barrier();

    // softmax role: thread (srow, sq) owns keys 4sq .. 4sq+3 of row srow; the row's 16 threads keep identical m, l
    const int srow = tid >> 4, sq = tid & 15;
    const int vis = min(nb + (srow >> 3), kend);  // row srow sees keys < vis (rows of absent tokens: < kend)
    float m_run = NEG_INF, l_run = 0.f;
    f32x16 O = f32x16{};

    // Q's B operands in registers for the whole loop (rows 16hb + lane%16, dims 128dh + 32s + 8(lane/16) .. +7): read
    // from LDS once here instead of in every stage, where a read behind the second row half's branch waited on the
    // one before
    half8 qb0[4], qb1[4], qbl0[EXACT ? 4 : 1], qbl1[EXACT ? 4 : 1];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        qb0[s] = *(const half8*)&qs[l16][128 * dh + 32 * s + 8 * g4];
        qb1[s] = *(const half8*)&qs[16 + l16][128 * dh + 32 * s + 8 * g4];
        if constexpr (EXACT) {
            qbl0[s] = *(const half8*)&qsl[l16][128 * dh + 32 * s + 8 * g4];
            qbl1[s] = *(const half8*)&qsl[16 + l16][128 * dh + 32 * s + 8 * g4];
        }
    }

    // S partial of this wave's 16 keys x 32 rows over its 128 dims, into ss[buf][dh]
    auto s_part = [&](int j, const StageRegs& R, int buf) {
        half8 kk[4] = {R.k[0], R.k[1], R.k[2], R.k[3]};
        const int k0 = kbase(j);
        if (k0 < apl && k0 + KPS > apf) {  // the stage holds new rows: their K from LDS
            const int key = k0 + kkey;
            if (key >= apf && key < apl) {
#pragma unroll
                for (int s = 0; s < 4; s++) kk[s] = *(const half8*)&newk[key - apf][128 * dh + 32 * s + 8 * g4];
            }
        }
        f32x4 s4[2] = {f32x4{}, f32x4{}};
#pragma unroll
        for (int s = 0; s < 4; s++) {
            s4[0] = mfma16(kk[s], qb0[s], s4[0]);
            if (ntb > 2) s4[1] = mfma16(kk[s], qb1[s], s4[1]);
            if constexpr (EXACT) {
                s4[0] = mfma16(kk[s], qbl0[s], s4[0]);
                if (ntb > 2) s4[1] = mfma16(kk[s], qbl1[s], s4[1]);
            }
        }
        return [&, s4, buf]() {
#pragma unroll
            for (int hb = 0; hb < 2; hb++)
                *(f32x4*)&ss[buf][dh][16 * hb + l16][16 * kq + 4 * g4] = s4[hb];
        };
    };

    // online softmax of stage j with the lazy reference max of attn_dmx (dmx.rs:72-86), log2 units: reads ss[buf],
    // writes P (f16) to ps[buf] and the rows' rescale factors to cfs[buf]
    auto softmax = [&](int j, int buf) {
        const int k0 = kbase(j);
        const float4 x0 = *(const float4*)&ss[buf][0][srow][4 * sq];
        const float4 x1 = *(const float4*)&ss[buf][1][srow][4 * sq];
        float sv[4] = {(x0.x + x1.x) * scale2, (x0.y + x1.y) * scale2, (x0.z + x1.z) * scale2, (x0.w + x1.w) * scale2};
        const int kcap = k0 + klen(j);
        if (!(k0 >= start && kcap <= nb && kcap == k0 + KPS)) {  // the stage crosses a row's window or is a half
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = k0 + 4 * sq + i;
                if (!(key < vis && key >= start && key < kcap)) sv[i] = NEG_INF;
            }
        }
        float mt = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        mt = reduce16(mt, [](float a, float b) { return fmaxf(a, b); });
        float mr = m_run;
        if (m_run == NEG_INF || mt > m_run + LAZY2) mr = fmaxf(m_run, mt);
        const float cf = m_run == NEG_INF ? 1.f : fast_exp2(m_run - mr);
        const float base = mr == NEG_INF ? 0.f : mr;  // masked scores are -inf: 2^-inf = 0
        float psum;
        if constexpr (EXACT) {  // f32 P: its hi and lo f16 parts for the matrix units, the f32 values for the sum
            const f32x4 pf = {fast_exp2(sv[0] - base), fast_exp2(sv[1] - base), fast_exp2(sv[2] - base),
                              fast_exp2(sv[3] - base)};
            psum = (pf.x + pf.y) + (pf.z + pf.w);
            half4 hi, lo;
            split4(pf, hi, lo);
            *(half4*)&ps[buf][srow][4 * sq] = hi;
            *(half4*)&psl[buf][srow][4 * sq] = lo;
        } else {
            typedef _Float16 half2v __attribute__((ext_vector_type(2)));
            const half2v p01 = {(_Float16)fast_exp2(sv[0] - base), (_Float16)fast_exp2(sv[1] - base)};
            const half2v p23 = {(_Float16)fast_exp2(sv[2] - base), (_Float16)fast_exp2(sv[3] - base)};
            const half2v one2 = {(_Float16)1.f, (_Float16)1.f};
            // l adds the f16-rounded P, summed in f32 (v_dot2_f32_f16 is exact for these products by 1)
            psum = __builtin_amdgcn_fdot2(p23, one2, __builtin_amdgcn_fdot2(p01, one2, 0.f, false), false);
            *(uint2*)&ps[buf][srow][4 * sq] =
                uint2{__builtin_bit_cast(unsigned, p01), __builtin_bit_cast(unsigned, p23)};
        }
        psum = reduce16(psum, [](float a, float b) { return a + b; });
        l_run = l_run * cf + psum;
        m_run = mr;
        if (sq == 0) cfs[buf][srow] = cf;
    };

    // O (this wave's 32 dims of the 32 rows) = O * cf + P . V of stage j
    auto pv = [&](int j, int buf, const StageRegs& R) {
        const int k0 = kbase(j);
        half8 pa[KPS / 16];
#pragma unroll
        for (int s2 = 0; s2 < KPS / 16; s2++) pa[s2] = *(const half8*)&ps[buf][r][16 * s2 + 8 * h];
        if (__any(cfs[buf][r] != 1.f)) {
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const float4 f = *(const float4*)&cfs[buf][8 * a + 4 * h];
                O[4 * a] *= f.x;
                O[4 * a + 1] *= f.y;
                O[4 * a + 2] *= f.z;
                O[4 * a + 3] *= f.w;
            }
        }
        half8 vb[KPS / 16] = {R.v[0], R.v[1], R.v[2], R.v[3]};
        if (k0 < apl && k0 + KPS > apf) {  // the stage holds new rows: their V from LDS
#pragma unroll
            for (int s2 = 0; s2 < KPS / 16; s2++) {
                if (k0 + 16 * s2 >= apl || k0 + 16 * s2 + 16 <= apf) continue;  // no new row in these 16 keys
                _Float16 x[8];  // all reads first (clamped rows), then the selects: no LDS round trip per key
#pragma unroll
                for (int jj = 0; jj < 8; jj++)
                    x[jj] = newv[min(max(k0 + 16 * s2 + 8 * h + jj - apf, 0), nr - 1)][32 * w + r];
#pragma unroll
                for (int jj = 0; jj < 8; jj++) {
                    const int key = k0 + 16 * s2 + 8 * h + jj;
                    if (key >= apf && key < apl) vb[s2][jj] = x[jj];
                }
            }
        }
        if (k0 + KPS > kend) {  // V rows past the written length may hold anything: keep 0 * V finite
#pragma unroll
            for (int s2 = 0; s2 < KPS / 16; s2++)
#pragma unroll
                for (int jj = 0; jj < 8; jj++)
                    if (k0 + 16 * s2 + 8 * h + jj >= kend) vb[s2][jj] = (_Float16)0.f;
        }
#pragma unroll
        for (int s2 = 0; s2 < KPS / 16; s2++) {
            O = mfma32(pa[s2], vb[s2], O);
            if constexpr (EXACT) O = mfma32(*(const half8*)&psl[buf][r][16 * s2 + 8 * h], vb[s2], O);
        }
    };

    // Software pipeline, one barrier per stage. Iteration j: issue the loads of K for stage j + 2 and of V for stage
    // j + 1, the S MFMAs of stage j + 1 (K loaded one iteration ago; they run while the VALU does the softmax of stage
    // j, whose S the previous iteration left in LDS), store S of j + 1, barrier, then P.V of stage j (V loaded one
    // iteration ago): about one stage of bytes in flight, each operand a whole iteration ahead. Buffers alternate by
    // stage parity; a buffer is rewritten two stages after it was read, behind the barrier between.
    auto iter2 = [&](int j, StageRegs& Kn, const StageRegs& K1, StageRegs& Vn, const StageRegs& V0, auto has_next) {
        const int buf = j & 1;
        load_k(j + 2, Kn);
        load_v(j + 1, Vn);
        if constexpr (decltype(has_next)::value) {
            auto store_s = s_part(j + 1, K1, buf ^ 1);
            softmax(j, buf);
            store_s();
        } else {
            softmax(j, buf);
        }
        lds_barrier();
        pv(j, buf, V0);
    };
    if (nst > 0) {
        s_part(0, R0, 0)();
        lds_barrier();
    }
    using T = std::true_type;
    using F = std::false_type;
    int j = 0;
    for (; j + 2 < nst; j += 2) {
        iter2(j, R0, R1, R3, R2, T{});
        iter2(j + 1, R1, R0, R2, R3, T{});
    }
    if (nst - j == 1) {
        iter2(j, R0, R1, R3, R2, F{});
    } else if (nst - j == 2) {
        iter2(j, R0, R1, R3, R2, T{});
        iter2(j + 1, R1, R0, R2, R3, F{});
    }

    // the appended rows into the planes, for the launches that follow (stores issued here, behind no loads)
    if (nr > 0) {
        unsigned short* Ku = (unsigned short*)K;
        unsigned short* Vu = (unsigned short*)V;
        for (int it = tid; it < nr * 32; it += 512) {
            const int i = it >> 5, d0 = (it & 31) * 8;
            *(u16x8*)(Ku + k_off(apf + i, d0)) = *(const u16x8*)&newk[i][d0];
        }
        for (int it = tid; it < nr * HD; it += 512) {
            const int i = it / HD, d = it % HD;
            Vu[v_off(apf + i, d)] = __builtin_bit_cast(unsigned short, newv[i][d]);
        }
    }

    // partials: this wave's 32 dims of every row of a present token; m and l from the rows' softmax threads
    const int nrows = 8 * ntb;
    const int rz = kvh * rpk + 32 * zb;  // partial row of this block's row 0
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int ri = 8 * (i >> 2) + 4 * h + (i & 3);
        if (ri < nrows) part[((size_t)(rz + ri) * nch + c) * PART + PACC + 32 * w + r] = O[i];
    }
    if (sq == 0 && srow < nrows) {
        float* p = part + ((size_t)(rz + srow) * nch + c) * PART;
        p[0] = m_run;
        p[1] = l_run;
    }
}

// Merge of the split-K partials: work-group (token, head, quarter of the dims); its 256 threads are 16 chunk lanes x
// 16 dim lanes (4 dims each), so every chunk's 64 dims are one coalesced 256-byte read and all chunks are in flight at
// once; the 16 chunk lanes are then summed in LDS.
// H16: the output as f16 bits, rounded to nearest even (attn_gate16's pack2x16float, ops.wgsl:296-300), else f32.
template <int MERGE_J, bool H16>  // chunks per chunk lane: 9 for up to 144 splits, 16 for up to 256
__global__ void __launch_bounds__(256) decode_combine(const float* __restrict__ part, int rpk, int n, int start,
                                                      int span, int nch, const float* __restrict__ gate,
                                                      void* __restrict__ out) {
    const int t = blockIdx.x / QH, head = blockIdx.x % QH, dq = blockIdx.y, tid = threadIdx.x;
    const int kvh = head / GQA, row = t * GQA + head % GQA;
    const float* p = part + ((size_t)kvh * rpk + row) * nch * PART;
    // the gate logit of this thread's output dim, loaded with the partials (one round trip for both)
    const float gl = gate && tid < 64 ? gate[((size_t)t * QH + head) * 512 + 256 + dq * 64 + tid] : 0.f;
    int c0, c1;  // chunks holding a key of [start, n + t)
    chunk_range(start, n + t, span, nch, c0, c1);
    __shared__ float red[4];
    __shared__ float4 acc4[16][16];
    __shared__ float redl[16];
    // one round trip: every thread loads all its chunks (at most MERGE_J) before using any
    const int cl = tid >> 4, dl = tid & 15;
    const int d0 = dq * 64 + dl * 4;
    float mj[MERGE_J], lj[MERGE_J];
    float4 aj[MERGE_J];
    float M = NEG_INF;
#pragma unroll
    for (int j = 0; j < MERGE_J; j++) {
        const int c = c0 + cl + 16 * j;
        mj[j] = NEG_INF;
        lj[j] = 0.f;
        aj[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c < c1) {
            const float* pc = p + (size_t)c * PART;
            mj[j] = pc[0];
            lj[j] = pc[1];
            aj[j] = *(const float4*)(pc + PACC + d0);
        }
        M = fmaxf(M, mj[j]);
    }
    // the wave's maximum: within each 16-lane row by DPP, then across rows (one LDS permute, one lane-half swap)
    M = reduce16(M, [](float a, float b) { return fmaxf(a, b); });
    M = max_xor32(fmaxf(M, __shfl_xor(M, 16)));
    if ((tid & 63) == 0) red[tid >> 6] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float L = 0.f;
#pragma unroll
    for (int j = 0; j < MERGE_J; j++) {
        const float e = mj[j] == NEG_INF ? 0.f : exp2f(mj[j] - M);
        L += e * lj[j];
        acc.x += e * aj[j].x;
        acc.y += e * aj[j].y;
        acc.z += e * aj[j].z;
        acc.w += e * aj[j].w;
    }
    acc4[cl][dl] = acc;
    if (dl == 0) redl[cl] = L;
    __syncthreads();
    if (tid < 64) {
        // thread = (dim 4 dd + comp): its component of every chunk lane's sum at one constant stride, so the 16
        // LDS reads are independent and issue together (a component chosen from a whole float4 read made a chain)
        const int dd = tid >> 2, comp = tid & 3;
        const float* col = &acc4[0][dd].x + comp;
        float sum = 0.f, lt = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            sum += col[i * 64];
            lt += redl[i];
        }
        const int d = dq * 64 + tid;
        float o = sum / lt;
        if (gate) o = o * (1.f / (1.f + expf(-gl)));
        const size_t oi = ((size_t)t * QH + head) * HD + d;
        if constexpr (H16) ((unsigned short*)out)[oi] = f2h(o);
        else ((float*)out)[oi] = o;
    }
}

// Merge for few chunks (prefill splits): a work-group of 256 threads merges 4 rows (token, head), 64 threads per
// row, 4 dims per thread (16-byte loads); every group of MERGE_FEW chunks of the row is loaded in one round trip.
template <bool GROUPS, bool H16, int NJ>  // GROUPS false: at most NJ chunks, one group; H16 as decode_combine
__global__ void __launch_bounds__(256) merge_few(const float* __restrict__ part, int rpk, int ntok, int n, int start,
                                                 int span, int nch, const float* __restrict__ gate,
                                                 void* __restrict__ out) {
    const int rowid = blockIdx.x * 4 + (threadIdx.x >> 6);  // t * 16 + head
    if (rowid >= ntok * QH) return;
    const int t = rowid / QH, head = rowid % QH, d0 = (threadIdx.x & 63) * 4;
    const int kvh = head / GQA, row = t * GQA + head % GQA;
    const float* p = part + ((size_t)kvh * rpk + row) * nch * PART;
    int c0, c1;  // chunks holding a key of [start, n + t)
    chunk_range(start, n + t, span, nch, c0, c1);
    // the gate logits of this thread's 4 output dims, loaded with the partials (one round trip for both)
    const float4 gl = gate ? *(const float4*)(gate + ((size_t)t * QH + head) * 512 + 256 + d0)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
    // the row's chunks in groups of MERGE_FEW, each group loaded in one round trip and folded into a running
    // (maximum, sum, accumulator); with one group this is the plain max-then-sum of the partials
    float M = NEG_INF, L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int g0 = c0; GROUPS ? g0 < c1 : g0 == c0; g0 += NJ) {
        float mj[NJ], lj[NJ];
        float4 aj[NJ];
        float Mg = NEG_INF;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int c = g0 + j;
            mj[j] = NEG_INF;
            lj[j] = 0.f;
            aj[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (c < c1) {
                const float* pc = p + (size_t)c * PART;
                mj[j] = pc[0];
                lj[j] = pc[1];
                aj[j] = *(const float4*)(pc + PACC + d0);
            }
            Mg = fmaxf(Mg, mj[j]);
        }
        const float Mn = fmaxf(M, Mg);
        const float sc = M == NEG_INF ? 0.f : exp2f(M - Mn);  // the groups before, to the new maximum
        L *= sc;
        acc.x *= sc;
        acc.y *= sc;
        acc.z *= sc;
        acc.w *= sc;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const float e = mj[j] == NEG_INF ? 0.f : exp2f(mj[j] - Mn);
            L += e * lj[j];
            acc.x += e * aj[j].x;
            acc.y += e * aj[j].y;
            acc.z += e * aj[j].z;
            acc.w += e * aj[j].w;
        }
        M = Mn;
    }
    float4 o = make_float4(acc.x / L, acc.y / L, acc.z / L, acc.w / L);
    if (gate) {
        o.x *= 1.f / (1.f + expf(-gl.x));
        o.y *= 1.f / (1.f + expf(-gl.y));
        o.z *= 1.f / (1.f + expf(-gl.z));
        o.w *= 1.f / (1.f + expf(-gl.w));
    }
    const size_t oi = ((size_t)t * QH + head) * HD + d0;
    if constexpr (H16) {
        const unsigned lo = f2h(o.x) | (unsigned)f2h(o.y) << 16, hi = f2h(o.z) | (unsigned)f2h(o.w) << 16;
        *(uint2*)((unsigned short*)out + oi) = make_uint2(lo, hi);
    } else {
        *(float4*)((float*)out + oi) = o;
    }
}

}  // namespace

DecodePlan decode_plan(int n, int ntok, int start) {
    // 64-position stages dealt round robin (neighbouring stages stream from different CUs at once, which keeps HBM
    // busier than one contiguous range per work-group), at most DEC_WG work-groups per kv head. Up to DEC_WG stages,
    // nu / 2 + 1 work-groups take two stages each but one or two of them, the last of which takes the stage holding
    // the appended rows (with one stage each, that work-group's append work came on top of a full share): 4 tokens at
    // 2,048 / 4,096 / 5,632 / 6,850 positions 9.7 / 10.0 / 10.4 / 10.8 us per step against 9.9 / 10.7 / 11.3 / 11.9,
    // 1 token at 4,097 (cfg1) 9.0 against 9.1 us. Under 32 stages, one stage each: too few work-groups stream
    // otherwise (4 tokens at 1,024 / 1,536 positions, two stages each: 9.7 / 10.1 against 9.6 / 9.8 us).
    const int kend = n + ntok - 1;
    const int s0 = start / KPS_F16 * KPS_F16;
    const int nu = (kend - s0 + KPS_F16 - 1) / KPS_F16;
    int g = nu >= 32 && nu <= DEC_WG ? nu / 2 + 1 : nu;
    g = g < 1 ? 1 : g > DEC_WG ? DEC_WG : g;
    return DecodePlan{0, g, 0, s0, nu};
}

hipError_t launch_decode_core(const Geom& g, void* base, int layer, const float* q, int ntok, int n, int start,
                              float scale, const DecodePlan& p, const DecodeWs& ws, const FusedAppend& fa,
                              const Launch& L) {
    if (p.nch > ws.max_chunks || p.nch - p.c0 > 16 * MERGE_JMAX) return hipErrorInvalidValue;
    char* b = (char*)base;
    void* kp = b + g.plane(layer, 0, 0) * g.plane_bytes();
    void* vp = b + g.plane(layer, 1, 0) * g.plane_bytes();
    const float scale2 = scale * LOG2E;
    if (g.fmt != 0 || ntok > 4) return hipErrorNotSupported;
    return launch(ntok == 1 || start > 0 ? decode_f16<true> : decode_f16<false>, dim3(p.nch, KVH), dim3(512), L, kp, vp,
                  g.plane_elems, q, ntok, n, start, scale2,
                  p.s0, p.nu, ws.part, fa.kn, fa.v, fa.tab, fa.pos, fa.ntok, ROWS, 0);
}

SmallPlan small_prefill_plan(int T, int n, int start) {
    // the decode's stages over the whole block's keys; at most SMALL_WG work-groups per (kv head, 4-token block) and
    // about SMALL_WG in all per kv head once there are several blocks (each block streams every stage)
    const int nzb = (T + 3) / 4;
    DecodePlan d = decode_plan(n, T, start);
    const int kend = n + T - 1, nu = (kend - d.s0 + KPS_F16 - 1) / KPS_F16;
    d.nch = min(max(nu, 1), SMALL_WG);
    const int cap = max(8, SMALL_WG / nzb);  // twice or four times as many splits measured slower
    d.nch = min(d.nch, cap);
    return SmallPlan{d, nzb};
}

size_t small_prefill_ws_floats(int T, int nch) { return (size_t)KVH * 32 * ((T + 3) / 4) * nch * PART; }

hipError_t launch_small_prefill(const Geom& g, const void* base, int layer, const float* q, int T, int n, int start,
                                float scale, const SmallPlan& p, float* ws, const Launch& L) {
    if (g.fmt != 0 || T < 1 || T > SMALL_PREFILL_MAX) return hipErrorNotSupported;
    char* b = (char*)base;
    void* kp = b + g.plane(layer, 0, 0) * g.plane_bytes();
    void* vp = b + g.plane(layer, 1, 0) * g.plane_bytes();
    const float scale2 = scale * LOG2E;
    // a 1D grid, XCD-aware with the token blocks fastest (the columns that stream a stage share an L2): 24.2 against
    // 28.2 us for 8 tokens and 51.8 against 57.9 us for 32 at 28,000 positions
    return launch(decode_f16<true>, dim3(p.d.nch * KVH * p.nzb), dim3(512), L, kp, vp, g.plane_elems, q, T, n, start,
                  scale2, p.d.s0, p.d.nu, ws, (const float*)nullptr, (const float*)nullptr, (const float*)nullptr, 0, 0,
                  32 * p.nzb, p.nzb);
}

template <bool H16>
hipError_t merge_as(const float* part, int rpk, int ntok, int n, int start, int span, int nch, const float* gate,
                    void* out, const Launch& L) {
    if (nch > 16 * MERGE_JMAX) return hipErrorInvalidValue;
    // few chunks, or many rows (prefill blocks) over up to two groups of chunks: a row per 64 threads (a 128-token
    // block at 28,000 positions, 32 splits, 87.8 against 94.2 us per step; with 64 splits, four groups, slower than
    // decode_combine: 68.4 against 63.0 us)
    const dim3 few((ntok * QH + 3) / 4), rows(ntok * QH, HD / 64);
    if (nch <= 8)  // the 8 splits of a 512-token block: 12.2 against 14.5 us with the 16-chunk build
        return launch(merge_few<false, H16, 8>, few, dim3(256), L, part, rpk, ntok, n, start, span, nch, gate, out);
    if (nch <= MERGE_FEW)
        return launch(merge_few<false, H16, MERGE_FEW>, few, dim3(256), L, part, rpk, ntok, n, start, span, nch, gate,
                      out);
    if (ntok >= 32 && nch <= 2 * MERGE_FEW)
        return launch(merge_few<true, H16, MERGE_FEW>, few, dim3(256), L, part, rpk, ntok, n, start, span, nch, gate,
                      out);
    if (nch <= 16 * 9)
        return launch(decode_combine<9, H16>, rows, dim3(256), L, part, rpk, n, start, span, nch, gate, out);
    return launch(decode_combine<MERGE_JMAX, H16>, rows, dim3(256), L, part, rpk, n, start, span, nch, gate, out);
}

hipError_t launch_merge(const float* part, int rpk, int ntok, int n, int start, int span, int nch, const float* gate,
                        void* out, bool h16, const Launch& L) {
    return h16 ? merge_as<true>(part, rpk, ntok, n, start, span, nch, gate, out, L)
               : merge_as<false>(part, rpk, ntok, n, start, span, nch, gate, out, L);
}

hipError_t launch_decode_merge(int ntok, int n, int start, const DecodePlan& p, const DecodeWs& ws, const float* gate,
                               void* out, bool h16, const Launch& L) {
    return launch_merge(ws.part, ROWS, ntok, n, start, p.span, p.nch, gate, out, h16, L);
}

}  // namespace mkv
