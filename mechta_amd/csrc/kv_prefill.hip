// kv_prefill.hip -- causal prefill flash attention on f16 MFMA, split-K over positions.
//
// Replaces q_f16 + attn_fa_mx + attn_fd_combine of the reference's prefill (fa_mx.wgsl:19-115, 313-319;
// engine.rs:1215-1236). Token t of the block (0-based) sees positions [start, n + t).
//
// Work-group = (32 tokens of the block, split of `ch` positions, kv head): 8 waves (two per SIMD, so one wave's
// softmax overlaps the other's matrix work), each owns 4 tokens x the kv head's 8 query heads = 32 query rows
// (row = token*8 + head). The split's 32-key tiles (a 16 KB K block and four 4 KB V groups, contiguous in HBM)
// stream through a 4-slot LDS ring filled by direct global->LDS loads, shared by the 8 waves. Per tile and wave:
//   S^T[32 keys][32 rows] = K . Q^T    16 x v_mfma_f32_32x32x16_f16 (A = K rows in key_perm order from LDS,
//                                      B = Q rounded to f16, held in registers for the whole split)
//   online softmax of the 32 rows in registers, lazy reference max (moves when first or when the tile max exceeds
//   it by more than 8), row sums from the f32 P (as attn_fa_mx), P rounded to f16 for the matrix units
//   O[32 rows][256] += P . V           16 x v_mfma_f32_32x32x16_f16 (A = P straight from the S registers,
//                                      B = V from LDS)
// Each wave writes one partial [m, l, acc[256]] per row; launch_merge combines the splits (and applies the gate).
#include "mkv_device.h"

namespace mkv {
namespace {

#ifndef MKV_PF_RB
#define MKV_PF_RB 1
#endif
#ifndef MKV_PF_NW
#define MKV_PF_NW 8
#endif
constexpr int RB = MKV_PF_RB;                 // 32-row blocks (4 tokens x 8 heads) per wave
constexpr int NW = MKV_PF_NW;                 // waves per work-group
constexpr int PT = NW * 4 * RB;               // tokens per work-group
constexpr int SUB = 1;                        // 32-key subtiles per ring slot (per barrier)
constexpr int TILE_BYTES = 32 * HD * 2;       // one 32-key K block (or its 4 V groups), f16
constexpr int SLOT_BYTES = 2 * SUB * TILE_BYTES;  // K blocks, then V groups of a slot
#ifndef MKV_PF_NSLOT
#define MKV_PF_NSLOT 4
#endif
#ifndef MKV_PF_WGS_PER_CU
#define MKV_PF_WGS_PER_CU 1
#endif
constexpr int NSLOT = MKV_PF_NSLOT;           // LDS ring slots: NSLOT - 1 tiles in flight while one is computed
constexpr int WGS_PER_CU = MKV_PF_WGS_PER_CU;  // work-groups the plan places per CU

constexpr int LPT = 2 * SUB * TILE_BYTES / NW / 1024;  // direct loads per slot and wave
static_assert(NSLOT == 2 || LPT == 4 || LPT == 8, "wait counts below");

__device__ inline void wait_tiles(int later) {  // at most `later` tiles (LPT direct loads each per wave) pending
    if constexpr (NSLOT == 2) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else if constexpr (LPT == 4) {
        if (later >= 2) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else if (later == 1) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
        if (later >= 2) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        else if (later == 1) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
}

__global__ void __launch_bounds__(NW * 64) prefill_f16(const _Float16* __restrict__ kplane,
                                                   const _Float16* __restrict__ vplane, size_t plane_elems,
                                                   const float* __restrict__ q, int T, int n, int start, float scale2,
                                                   int span, int nch, float* __restrict__ part) {
    // XCD-aware order: the dispatcher deals consecutive work-groups round robin to the 8 XCDs (each with its own
    // L2), so work item W = xcd * (grid / 8) + slot keeps the token blocks of one (split, kv head) -- the
    // work-groups that stream the same keys -- on one XCD, and each key is fetched into one L2 instead of eight.
    const int G = gridDim.x, L = blockIdx.x;
    const int W = G % NXCD == 0 ? (L % NXCD) * (G / NXCD) + L / NXCD : L;
    const int nblk = (T + PT - 1) / PT;
    const int rb = W % nblk, sp = (W / nblk) % nch, kvh = W / nblk / nch, tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int h = lane >> 5, r = lane & 31;
    const int t0 = rb * PT + 4 * RB * w;     // this wave's first token; row block b holds tokens t0 + 4b .. +3
    const int tlast = min(T - 1, rb * PT + PT - 1);
    const int kend = n + T - 1;              // positions written for this block
    const int cs = chunk_lo(sp, span, nch), ce = min(sp + 1 < nch ? chunk_lo(sp + 1, span, nch) : span, n + tlast);
    if (cs >= ce) return;                    // no key of this split is seen by these tokens: never merged
    const _Float16* K = kplane + (size_t)kvh * plane_elems;
    const _Float16* V = vplane + (size_t)kvh * plane_elems;

    __shared__ __attribute__((aligned(16))) unsigned char ring[NSLOT * SLOT_BYTES];
    __shared__ __attribute__((aligned(16))) float cfs[NW][32];  // rescale factors of a wave's rows
    const int ntiles = (ce - cs + 32 * SUB - 1) / (32 * SUB);
    constexpr int PART_BYTES = SUB * TILE_BYTES / NW;
    // the wave's part of a tile: a per-lane offset fixed for the kernel; the tile's base and LDS slot are wave-uniform
    const unsigned voff = w * PART_BYTES + lane * 16;
    const unsigned wlds = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_void*)ring + w * PART_BYTES);
    // V rows past the written length may hold anything: each wave zeroes them in the part of tile j it copied itself,
    // after its own copies have landed and before the barrier that hands the tile to every wave (no barrier of its own)
    auto zero_own_tail = [&](int j) {
        const int k0 = cs + 32 * SUB * j;
        if (k0 + 32 * SUB <= kend) return;
        unsigned char* Vw = ring + (j % NSLOT) * SLOT_BYTES + SUB * TILE_BYTES;
#pragma unroll
        for (int i = 0; i < PART_BYTES / 1024; i++) {
            const unsigned off = voff + i * 1024;  // 8 consecutive positions of one dim: group off / 4096
            const int key = k0 + (int)(off / 4096) * 8;
            if (key + 8 > kend) {
                half8 x = *(const half8*)(Vw + off);
#pragma unroll
                for (int e = 0; e < 8; e++)
                    if (key + e >= kend) x[e] = (_Float16)0.f;
                *(half8*)(Vw + off) = x;
            }
        }
    };
    auto issue = [&](int j) {  // each wave copies 1/NW of tile j's K blocks and V groups into slot j % NSLOT
        const int k0 = cs + 32 * SUB * j;
        const unsigned char* ks = (const unsigned char*)(K + (size_t)(k0 / KBLK) * (KBLK * HD));
        const unsigned char* vs = (const unsigned char*)(V + (size_t)(k0 / VGRP) * (VGRP * HD));
        const unsigned dst = wlds + (j % NSLOT) * SLOT_BYTES;
#pragma unroll
        for (int i = 0; i < PART_BYTES / 1024; i++) dma16s(ks + i * 1024, voff, dst + i * 1024);
#pragma unroll
        for (int i = 0; i < PART_BYTES / 1024; i++) dma16s(vs + i * 1024, voff, dst + SUB * TILE_BYTES + i * 1024);
    };
    for (int j = 0; j < NSLOT - 1 && j < ntiles; j++) issue(j);

    // Q as the B operand of S^T: for row block b, lane (r, h) holds row r (token t0 + 4b + r/8, head r%8), dims
    // 16s + 8h .. +7 for step s, rounded to f16 (q_f16); rows of tokens past the block are zero
    half8 qb[RB][16];
    int vis[RB];
#pragma unroll
    for (int b = 0; b < RB; b++) {
        const int tr = t0 + 4 * b + (r >> 3);
        vis[b] = tr < T ? n + tr : 0;  // row r of block b sees keys < vis[b]
        const float* qrow = q + ((size_t)min(tr, T - 1) * QH + kvh * GQA + (r & 7)) * HD + 8 * h;
#pragma unroll
        for (int s = 0; s < 16; s++) {
            float4 x0 = *(const float4*)(qrow + 16 * s), x1 = *(const float4*)(qrow + 16 * s + 4);
            if (tr >= T) x0 = x1 = make_float4(0.f, 0.f, 0.f, 0.f);
            qb[b][s] = half8{(_Float16)x0.x, (_Float16)x0.y, (_Float16)x0.z, (_Float16)x0.w,
                             (_Float16)x1.x, (_Float16)x1.y, (_Float16)x1.z, (_Float16)x1.w};
        }
    }
    const int kaddr = h * 512 + key_perm(r) * 16;
    // the smallest window end of each row block (its first token's; 0 when the block runs past T): a tile with every
    // key below it, and none below start, needs no mask (a wave-uniform test)
    int vmin[RB];
#pragma unroll
    for (int b = 0; b < RB; b++) {
        const int tf = __builtin_amdgcn_readfirstlane(t0 + 4 * b);
        vmin[b] = tf + 3 < T ? n + tf : 0;
    }
    float m[RB], lsum[RB];
    f32x16 O[RB][8];
#pragma unroll
    for (int b = 0; b < RB; b++) {
        m[b] = NEG_INF;
        lsum[b] = 0.f;
#pragma unroll
        for (int nb = 0; nb < 8; nb++) O[b][nb] = f32x16{};
    }

    // S of tile j, the mask where it crosses a row's window, the online softmax (lazy reference max, O rescaled when a
    // finite reference moved) and P into pa
    auto s_mfma = [&](int j, f32x16(&Scur)[RB]) {
        const unsigned char* Ks = ring + (j % NSLOT) * SLOT_BYTES;
#pragma unroll
        for (int b = 0; b < RB; b++) Scur[b] = f32x16{};
        constexpr int KP = 3;  // K operands in flight ahead of the S chain (LDS latency; 4 to 6 measured no faster)
        half8 kbuf[KP];
#pragma unroll
        for (int s = 0; s < KP; s++) kbuf[s] = *(const half8*)(Ks + kaddr + s * 1024);
#pragma unroll
        for (int s = 0; s < 16; s++) {
            const half8 ka = kbuf[s % KP];
            if (s + KP < 16) kbuf[s % KP] = *(const half8*)(Ks + kaddr + (s + KP) * 1024);
#pragma unroll
            for (int b = 0; b < RB; b++) Scur[b] = mfma32(ka, qb[b][s], Scur[b]);
        }
        // schedule: KP LDS reads (mask 0x100), then alternately one MFMA (0x008) and the next LDS read
        __builtin_amdgcn_sched_group_barrier(0x100, KP, 0);
#pragma unroll
        for (int s = 0; s < 16 - KP; s++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, KP, 0);
    };
    auto softmax = [&](int j, f32x16(&Scur)[RB], half8(&pa)[RB][2]) {
        const int k0 = cs + 32 * j;
#pragma unroll
        for (int b = 0; b < RB; b++) {
            // the causal / start mask only where this tile crosses a row's window (raw scores; the scale, log2
            // units, is applied to the max and inside the exponent's FMA)
            if (!(k0 >= start && k0 + 32 <= vmin[b])) {
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int key = k0 + 8 * h + i + (i >= 8 ? 8 : 0);
                    Scur[b][i] = (key < vis[b] && key >= start) ? Scur[b][i] : NEG_INF;
                }
            }
            // the first maximum is the compiler's: it reads the MFMA results and so carries the wait states a
            // vector read of them needs, which inline assembly would not get; the rest follows it
            float mt = fmaxf(Scur[b][0], Scur[b][1]);
#pragma unroll
            for (int i = 2; i < 16; i += 2) mt = vmax3(mt, Scur[b][i], Scur[b][i + 1]);
            mt = max_xor32(mt);
            mt *= scale2;  // scale2 > 0: the max of the scaled scores is the scaled max
            // the reference max moves when first or when the tile max exceeds it by more than 8; O and the sum are
            // rescaled only when a finite reference moved (rare: the exponential is not evaluated otherwise)
            const bool rescale = m[b] != NEG_INF && mt > m[b] + LAZY2;
            const float mr = m[b] == NEG_INF || rescale ? fmaxf(m[b], mt) : m[b];
            float cf = 1.f;
            if (__any(rescale)) {
                // register i of O holds row 8(i/4) + 4h + i%4, whose factor lane (that row) holds: the 32 factors pass
                // through this wave's LDS row (constant offsets, no per-register lane index to keep)
                cf = rescale ? fast_exp2(m[b] - mr) : 1.f;
                if (h == 0) cfs[w][r] = cf;
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int a = 0; a < 4; a++) {
                    const f32x4 f = *(const f32x4*)&cfs[w][8 * a + 4 * h];
#pragma unroll
                    for (int nb = 0; nb < 8; nb++) {
#pragma unroll
                        for (int q = 0; q < 4; q++) O[b][nb][4 * a + q] *= f[q];
                    }
                }
            }
            m[b] = mr;
            // P = 2^(s * scale2 - m) (one FMA): masked scores are -inf and give 0 (the reference is 0 while a row has seen no key);
            // the row sum takes the f32 P, as attn_fa_mx does, the P.V operand its f16 rounding
            const float base = mr == NEG_INF ? 0.f : mr;
            float ls;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float p = fast_exp2(__builtin_fmaf(Scur[b][i], scale2, -base));
                ls = i == 0 ? p : ls + p;  // 0 + p0 is p0: the same sum without the first add
                pa[b][i >> 3][i & 7] = (_Float16)p;
            }
            lsum[b] = lsum[b] * cf + ls;
        }
    };
    // O += P . V of tile j
    auto pv_tile = [&](int j, const half8(&pa)[RB][2]) {
        const unsigned char* Vs = ring + (j % NSLOT) * SLOT_BYTES + TILE_BYTES;
        constexpr int VP = 3;  // V operands in flight ahead of the P.V MFMAs
        half8 vbuf[VP];
        auto vaddr = [&](int i) { return Vs + (2 * (i >> 3) + h) * 4096 + (32 * (i & 7) + r) * 16; };
#pragma unroll
        for (int i = 0; i < VP; i++) vbuf[i] = *(const half8*)vaddr(i);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const half8 vb = vbuf[i % VP];
            if (i + VP < 16) vbuf[i % VP] = *(const half8*)vaddr(i + VP);
#pragma unroll
            for (int b = 0; b < RB; b++) O[b][i & 7] = mfma32(pa[b][i >> 3], vb, O[b][i & 7]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, VP, 0);
#pragma unroll
        for (int i = 0; i < 16 - VP; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, VP, 0);
    };
    for (int j = 0; j < ntiles; j++) {
        wait_tiles(min(ntiles - 1 - j, NSLOT - 2));
        zero_own_tail(j);
        lds_barrier();  // tile j is in LDS for every wave; every wave is done with tile j - 1
        if (j + NSLOT - 1 < ntiles) issue(j + NSLOT - 1);  // into the slot of tile j - 1
        f32x16 S[RB];
        half8 pa[RB][2];
        s_mfma(j, S);
        softmax(j, S, pa);
        pv_tile(j, pa);
    }

    // partials of this wave's rows of present tokens: row index t*8 + head of the kv head, rows per kv head = 8T
    const size_t rpk = (size_t)T * GQA;
#pragma unroll
    for (int b = 0; b < RB; b++) {
        lsum[b] += __shfl_xor(lsum[b], 32);
        const int tb = t0 + 4 * b;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int ri = 8 * (i >> 2) + 4 * h + (i & 3);
            if (tb + (ri >> 3) < T) {
                float* p = part + ((kvh * rpk + (size_t)tb * GQA + ri) * nch + sp) * PART + PACC + r;
#pragma unroll
                for (int nb = 0; nb < 8; nb++) p[32 * nb] = O[b][nb][i];
            }
        }
        if (h == 0 && tb + (r >> 3) < T) {
            float* p = part + ((kvh * rpk + (size_t)tb * GQA + r) * nch + sp) * PART;
            p[0] = m[b];
            p[1] = lsum[b];
        }
    }
}


// ---- f32 store: causal prefill with f32-class arithmetic (attn_fa, ops.wgsl:540-651) ----
// Work-group = (16 tokens of the block, key split, kv head), 8 waves: wave w takes row block w / 2 (4 tokens x 8
// heads = 32 rows) and dim half w % 2 (128 dims). The split's 32-key tiles (32 KB of K, 32 KB of V) stream through a
// 2-slot LDS ring filled by direct global->LDS loads and shared by the 8 waves, so a key is fetched once per 16
// tokens. f32 operands are split into f16 hi + lo (hi.hi + hi.lo + lo.hi on v_mfma_f32_32x32x16_f16). Per tile and
// wave:
//   partial S^T[32 keys][32 rows] over the wave's 128 dims: 8 dim steps x 3 passes (A = K rows in key_perm order,
//   the tile's K and V split into hi + lo once, in place in the ring, by the whole work-group; B = Q split once, in
//   registers); the two halves are exchanged through LDS and added
//   (a + b in both waves, so both hold the same S)
//   online softmax with a lazy reference max, redundantly in both waves of the pair
//   O[32 rows][the wave's 128 dims] += P . V: 2 key steps x 4 dim blocks x 3 passes
// Registers hold Q's hi and lo for 128 dims and O for 128 dims; LDS is 128 KB of ring and 32 KB of S exchange.
constexpr int P32_NW = 8;
constexpr int P32_PT = 16;                    // tokens per work-group
constexpr int P32_TILE = 32 * HD * 4;         // f32 K (or V) bytes of 32 positions: 32 KB
constexpr int P32_SLOT = 2 * P32_TILE;
constexpr int P32_LPT = P32_SLOT / P32_NW / 1024;  // direct loads per wave and slot: 8

__global__ void __launch_bounds__(P32_NW * 64) prefill_f32(const float* __restrict__ kplane,
                                                          const float* __restrict__ vplane, size_t plane_elems,
                                                          const float* __restrict__ q, int T, int n, int start,
                                                          float scale2, int span, int nch, float* __restrict__ part) {
    const int G = gridDim.x, Lb = blockIdx.x;
    const int W = G % NXCD == 0 ? (Lb % NXCD) * (G / NXCD) + Lb / NXCD : Lb;
    const int nblk = (T + P32_PT - 1) / P32_PT;
    const int rb = W % nblk, sp = (W / nblk) % nch, kvh = W / nblk / nch, tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, h = lane >> 5, r = lane & 31, blk = w >> 1, dh = w & 1;
    const int t0 = rb * P32_PT + 4 * blk;  // this wave's first token
    const int tlast = min(T - 1, rb * P32_PT + P32_PT - 1);
    const int kend = n + T - 1;            // positions written for this block
    const int cs = chunk_lo(sp, span, nch), ce = min(sp + 1 < nch ? chunk_lo(sp + 1, span, nch) : span, n + tlast);
    const int ntiles = ce > cs ? (ce - cs + 31) / 32 : 0;
    const unsigned char* K = (const unsigned char*)(kplane + (size_t)kvh * plane_elems);
    const unsigned char* V = (const unsigned char*)(vplane + (size_t)kvh * plane_elems);

    __shared__ __attribute__((aligned(16))) unsigned char ring[2 * P32_SLOT];
    __shared__ __attribute__((aligned(16))) f32x4 xs[P32_NW][4][64];  // each wave's partial S^T
    // Each wave copies 1/8 of tile j's K and V into slot j % 2, chosen so that the 16-byte chunk pairs it later splits
    // (below) are all its own: K bytes [4 KB w, +4 KB) (chunks d/4 = 8w .. 8w + 7 of every key), V dims
    // [128 (w % 2), +128) of groups 2 (w / 2) and 2 (w / 2) + 1 (2 KB each).
    const unsigned kreg = w * (P32_TILE / P32_NW);
    const unsigned vreg0 = (2 * (w >> 1)) * (HD * 16) + (w & 1) * (HD / 2 * 16), vreg1 = vreg0 + HD * 16;
    static_assert(P32_TILE / P32_NW == 4096 && HD / 2 * 16 == 2048, "4 KB of K and 2 x 2 KB of V per wave");
    // per-lane offsets of the wave's regions, fixed for the kernel; the tile's base and LDS slot are wave-uniform
    const unsigned vk = kreg + lane * 16, v0 = vreg0 + lane * 16, v1 = vreg1 + lane * 16;
    const unsigned lk = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_void*)ring + kreg);
    const unsigned l0 = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_void*)ring + P32_TILE + vreg0);
    const unsigned l1 = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_void*)ring + P32_TILE + vreg1);
    auto issue = [&](int j) {
        const size_t off = (size_t)(cs + 32 * j) * HD * 4;
        const unsigned slot = (j & 1) * P32_SLOT;
#pragma unroll
        for (int d = 0; d < 4; d++) dma16s(K + off + d * 1024, vk, lk + slot + d * 1024);
#pragma unroll
        for (int d = 0; d < 2; d++) {
            dma16s(V + off + d * 1024, v0, l0 + slot + d * 1024);
            dma16s(V + off + d * 1024, v1, l1 + slot + d * 1024);
        }
    };
    if (ntiles > 0) issue(0);

    // Q: lane (r, h) holds row r (token t0 + r / 8, head r % 8), dims 128dh + 16s + 8h .. +7 of step s, split
    const int tr = t0 + (r >> 3);
    const int vis = tr < T ? n + tr : 0;  // row r sees keys [start, vis)
    half8 qh[8], ql[8];
    {
        const float* qrow = q + ((size_t)min(tr, T - 1) * QH + kvh * GQA + (r & 7)) * HD + 128 * dh + 8 * h;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            f32x4 x0 = *(const f32x4*)(qrow + 16 * s), x1 = *(const f32x4*)(qrow + 16 * s + 4);
            if (tr >= T) x0 = x1 = f32x4{};
            split8(x0, x1, qh[s], ql[s]);
        }
    }
    const int kaddr = (32 * dh + 2 * h) * 512 + key_perm(r) * 16;  // K chunk (dims / 4) 32dh + 4s + 2h, +1
    float m = NEG_INF, lsum = 0.f;
    f32x16 O[4];
#pragma unroll
    for (int nb = 0; nb < 4; nb++) O[nb] = f32x16{};

    for (int j = 0; j < ntiles; j++) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's copies of tile j have landed
        const int k0 = cs + 32 * j;
        unsigned char* Ks = ring + (j & 1) * P32_SLOT;
        unsigned char* Vs = Ks + P32_TILE;
        // This wave's part of tile j split once, in place, into f16 hi + lo (the 4 row blocks' waves then read split
        // operands instead of each splitting the same tile): a pair of 16-byte chunks holds 8 consecutive dims of one
        // key (K chunks d/4 = 2g, 2g + 1) or 8 consecutive keys of one dim (V groups 2g, 2g + 1); hi goes over the
        // first chunk and lo over the second, where the operand reads below find them. The pairs are the ones this
        // wave copied, so no barrier comes between its copies and its split. V rows past the written length are
        // zeroed on the way (0 * V stays finite).
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int pk = lane + 64 * u;  // K pair pk: chunk 8w + 2 (pk / 32) of key pk % 32
            unsigned char* a = Ks + ((8 * w + 2 * (pk >> 5)) * 32 + (pk & 31)) * 16;
            half8 hi, lo;
            split8(*(const f32x4*)a, *(const f32x4*)(a + 512), hi, lo);
            unsigned char* b = Vs + vreg0 + (lane + 64 * u) * 16;  // V pair: dim 128 (w % 2) + lane + 64u
            f32x4 v0 = *(const f32x4*)b, v1 = *(const f32x4*)(b + HD * 16);
            if (k0 + 32 > kend) {
                const int key = k0 + 8 * (w >> 1);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    v0[e] = key + e < kend ? v0[e] : 0.f;
                    v1[e] = key + 4 + e < kend ? v1[e] : 0.f;
                }
            }
            half8 vh, vl;
            split8(v0, v1, vh, vl);
            *(half8*)a = hi;
            *(half8*)(a + 512) = lo;
            *(half8*)b = vh;
            *(half8*)(b + HD * 16) = vl;
        }
        lds_barrier();  // tile j is in LDS, split, for every wave; every wave is done with tile j - 1 and its exchange
        if (j + 1 < ntiles) issue(j + 1);  // into the slot of tile j - 1
        f32x16 Sh = f32x16{}, Sl = f32x16{};
        constexpr int KP = 2;
        half8 kb[KP][2];
#pragma unroll
        for (int s = 0; s < KP; s++) {
            kb[s][0] = *(const half8*)(Ks + kaddr + s * 2048);
            kb[s][1] = *(const half8*)(Ks + kaddr + s * 2048 + 512);
        }
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const half8 kh = kb[s % KP][0], kl = kb[s % KP][1];
            if (s + KP < 8) {
                kb[s % KP][0] = *(const half8*)(Ks + kaddr + (s + KP) * 2048);
                kb[s % KP][1] = *(const half8*)(Ks + kaddr + (s + KP) * 2048 + 512);
            }
            Sh = mfma32(kh, qh[s], Sh);
            Sl = mfma32(kh, ql[s], Sl);
            Sl = mfma32(kl, qh[s], Sl);
        }
        f32x16 S = Sh + Sl;
#pragma unroll
        for (int a = 0; a < 4; a++) xs[w][a][lane] = f32x4{S[4 * a], S[4 * a + 1], S[4 * a + 2], S[4 * a + 3]};
        lds_barrier();
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const f32x4 o = xs[w ^ 1][a][lane];
#pragma unroll
            for (int b = 0; b < 4; b++) S[4 * a + b] += o[b];  // a + b == b + a: both waves hold the same S
        }
        // register i of lane (r, h) is key 8h + i (i < 8) or 16 + 8h + i - 8 of the tile for row r
        if (!__all(k0 >= start && k0 + 32 <= vis)) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int key = k0 + 8 * h + i + (i >= 8 ? 8 : 0);
                S[i] = (key >= start && key < vis) ? S[i] : NEG_INF;
            }
        }
        float mt = vmax(S[0], S[1]);  // masked scores are -inf, never NaN: single-instruction maxima
#pragma unroll
        for (int i = 2; i < 16; i += 2) mt = vmax3(mt, S[i], S[i + 1]);
        mt = max_xor32(mt);
        mt *= scale2;  // scale2 > 0
        const bool rescale = m != NEG_INF && mt > m + LAZY2;
        const float mr = m == NEG_INF || rescale ? fmaxf(m, mt) : m;
        float cf = 1.f;
        if (__any(rescale)) {  // register i of O holds row 8(i/4) + 4h + i%4, whose factor that row's lanes hold
            cf = rescale ? fast_exp2(m - mr) : 1.f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float f = __shfl(cf, 8 * (i >> 2) + 4 * h + (i & 3));
#pragma unroll
                for (int nb = 0; nb < 4; nb++) O[nb][i] *= f;
            }
        }
        m = mr;
        const float base = mr == NEG_INF ? 0.f : mr;
        float p[16], ls = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            p[i] = fast_exp2(__builtin_fmaf(S[i], scale2, -base));
            ls += p[i];
        }
        lsum = lsum * cf + ls;
        half8 ph[2], pl[2];
#pragma unroll
        for (int k = 0; k < 2; k++)
            split8(f32x4{p[8 * k], p[8 * k + 1], p[8 * k + 2], p[8 * k + 3]},
                   f32x4{p[8 * k + 4], p[8 * k + 5], p[8 * k + 6], p[8 * k + 7]}, ph[k], pl[k]);
        // key step k: keys 16k + 8h .. +7 = V groups 4k + 2h, +1; dim block nb: dims 128dh + 32nb + r
        auto vaddr = [&](int i) { return Vs + ((4 * (i >> 2) + 2 * h) * HD + 128 * dh + 32 * (i & 3) + r) * 16; };
        constexpr int VP = 2;
        half8 vb[VP][2];
#pragma unroll
        for (int i = 0; i < VP; i++) {
            vb[i][0] = *(const half8*)vaddr(i);
            vb[i][1] = *(const half8*)(vaddr(i) + HD * 16);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const half8 vh = vb[i % VP][0], vl = vb[i % VP][1];
            if (i + VP < 8) {
                vb[i % VP][0] = *(const half8*)vaddr(i + VP);
                vb[i % VP][1] = *(const half8*)(vaddr(i + VP) + HD * 16);
            }
            O[i & 3] = mfma32(pl[i >> 2], vh, mfma32(ph[i >> 2], vl, mfma32(ph[i >> 2], vh, O[i & 3])));
        }
    }

    // partials of this wave's rows of present tokens: its 128 dims; m and l from the dim-half-0 wave
    lsum += __shfl_xor(lsum, 32);
    const size_t rpk = (size_t)T * GQA;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int ri = 8 * (i >> 2) + 4 * h + (i & 3);
        if (t0 + (ri >> 3) < T) {
            float* pp = part + ((kvh * rpk + (size_t)t0 * GQA + ri) * nch + sp) * PART + PACC + 128 * dh + r;
#pragma unroll
            for (int nb = 0; nb < 4; nb++) pp[32 * nb] = O[nb][i];
        }
    }
    if (dh == 0 && h == 0 && tr < T) {
        float* pp = part + ((kvh * rpk + (size_t)t0 * GQA + r) * nch + sp) * PART;
        pp[0] = m;
        pp[1] = lsum;
    }
}

}  // namespace

// Splits per prefill plan at most: about one work-group per CU down to blocks of 64 tokens (f16) or 5 (f32); with
// at most 16, a 64-token block at 28,000 positions took 95 us on 64 work-groups, now 64 us on 256 (f32 store: 16
// tokens 197 -> 65 us). The workspace bound, tokens x splits <= 4,096, is unchanged.
constexpr int PF_MAXCH = 64;
PrefillPlan prefill_plan(int T, int n) {
    const int kend = n + T - 1;
    const int blocks = 2 * ((T + PT - 1) / PT);  // work-groups per split
    int nch = 256 * WGS_PER_CU / blocks;         // about WGS_PER_CU work-groups per CU
    const int most = kend / 64;                  // splits of at least 64 positions
    nch = nch > most ? most : nch;
    nch = nch < 1 ? 1 : nch > PF_MAXCH ? PF_MAXCH : nch;
    return PrefillPlan{kend, nch};
}

PrefillPlan prefill32_plan(int T, int n) {
    const int kend = n + T - 1;
    const int blocks = KVH * ((T + P32_PT - 1) / P32_PT);  // work-groups per split
    int nch = 256 / blocks;                               // about one work-group per CU
    const int most = kend / 64;                           // splits of at least 64 positions
    nch = nch > most ? most : nch;
    nch = nch < 1 ? 1 : nch > PF_MAXCH ? PF_MAXCH : nch;
    return PrefillPlan{kend, nch};
}

size_t prefill_ws_floats(int T, int nch) { return (size_t)KVH * T * GQA * nch * PART; }

hipError_t launch_prefill(const Geom& g, const void* base, int layer, const float* q, int T, int n, int start,
                          float scale, const PrefillPlan& p, float* ws, const Launch& L) {
    if (g.fmt != 0) return hipErrorNotSupported;
    const char* b = (const char*)base;
    const void* kp = b + g.plane(layer, 0, 0) * g.plane_bytes();
    const void* vp = b + g.plane(layer, 1, 0) * g.plane_bytes();
    dim3 grid((T + PT - 1) / PT * p.nch * KVH);
    return launch(prefill_f16, grid, dim3(NW * 64), L, kp, vp, g.plane_elems, q, T, n, start, scale * LOG2E, p.span,
                  p.nch, ws);
}

hipError_t launch_prefill_f32(const Geom& g, const void* base, int layer, const float* q, int T, int n, int start,
                              float scale, const PrefillPlan& p, float* ws, const Launch& L) {
    if (g.fmt != 1) return hipErrorNotSupported;
    const char* b = (const char*)base;
    const float* kp = (const float*)(b + g.plane(layer, 0, 0) * g.plane_bytes());
    const float* vp = (const float*)(b + g.plane(layer, 1, 0) * g.plane_bytes());
    dim3 grid((T + P32_PT - 1) / P32_PT * p.nch * KVH);
    return launch(prefill_f32, grid, dim3(P32_NW * 64), L, kp, vp, g.plane_elems, q, T, n, start, scale * LOG2E,
                  p.span, p.nch, ws);
}

}  // namespace mkv
