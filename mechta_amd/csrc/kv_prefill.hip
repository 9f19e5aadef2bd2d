// kv_prefill.hip -- causal prefill flash attention on f16 MFMA, split-K over positions.
//
// Replaces q_f16 + attn_fa_mx + attn_fd_combine of the reference's prefill (fa_mx.wgsl:19-115, 313-319;
// engine.rs:1215-1236). Token t of the block (0-based) sees positions [start, n + t).
//
// Work-group = (16 tokens of the block, split of `ch` positions, kv head): 4 waves, each owns 4 tokens x the kv
// head's 8 query heads = 32 query rows (row = token*8 + head). The split's 32-key tiles (a 16 KB K block and four
// 4 KB V groups, contiguous in HBM) stream through a 4-slot LDS ring filled by direct global->LDS loads, shared by
// the 4 waves. Per tile and wave:
//   S^T[32 keys][32 rows] = K . Q^T    16 x v_mfma_f32_32x32x16_f16 (A = K rows in key_perm order from LDS,
//                                      B = Q rounded to f16, held in registers for the whole split)
//   online softmax of the 32 rows in registers, lazy reference max (moves when first or when the tile max exceeds
//   it by more than 8), P rounded to f16
//   O[32 rows][256] += P . V           16 x v_mfma_f32_32x32x16_f16 (A = P straight from the S registers,
//                                      B = V from LDS)
// Each wave writes one partial [m, l, acc[256]] per row; launch_merge combines the splits (and applies the gate).
#include "mkv_device.h"

namespace mkv {
namespace {

constexpr int PT = 16;                        // tokens per work-group
constexpr int TILE_BYTES = 32 * HD * 2;       // one 32-key K block (or its 4 V groups), f16
constexpr int SLOT_BYTES = 2 * TILE_BYTES;    // K + V of a tile
constexpr int NSLOT = 4;                      // LDS ring: 3 tiles in flight while one is computed

__device__ inline void wait_tiles(int later) {  // at most `later` tiles (8 direct loads each) still pending
    if (later >= 2) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else if (later == 1) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

__global__ void __launch_bounds__(256) prefill_f16(const _Float16* __restrict__ kplane,
                                                   const _Float16* __restrict__ vplane, size_t plane_elems,
                                                   const float* __restrict__ q, int T, int n, int start, float scale2,
                                                   int ch, int nch, float* __restrict__ part) {
    const int rb = blockIdx.x, sp = blockIdx.y, kvh = blockIdx.z, tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int h = lane >> 5, r = lane & 31;
    const int t0 = rb * PT + 4 * w;          // this wave's first token
    const int tlast = min(T - 1, rb * PT + PT - 1);
    const int kend = n + T - 1;              // positions written for this block
    const int cs = sp * ch, ce = min(cs + ch, n + tlast);
    if (cs >= ce) return;                    // no key of this split is seen by these tokens: never merged
    const _Float16* K = kplane + (size_t)kvh * plane_elems;
    const _Float16* V = vplane + (size_t)kvh * plane_elems;

    __shared__ __attribute__((aligned(16))) unsigned char ring[NSLOT * SLOT_BYTES];
    const int ntiles = (ce - cs + 31) / 32;
    auto issue = [&](int j) {  // each wave copies a quarter of tile j's K block and V groups into slot j % NSLOT
        const int k0 = cs + 32 * j;
        const unsigned char* ks = (const unsigned char*)(K + (size_t)(k0 / KBLK) * (KBLK * HD)) + w * 4096 + lane * 16;
        const unsigned char* vs = (const unsigned char*)(V + (size_t)(k0 / VGRP) * (VGRP * HD)) + w * 4096 + lane * 16;
        unsigned char* dst = ring + (j % NSLOT) * SLOT_BYTES + w * 4096;
#pragma unroll
        for (int i = 0; i < 4; i++) dma16(ks + i * 1024, dst + i * 1024);
#pragma unroll
        for (int i = 0; i < 4; i++) dma16(vs + i * 1024, dst + TILE_BYTES + i * 1024);
    };
    for (int j = 0; j < NSLOT - 1 && j < ntiles; j++) issue(j);

    // Q as the B operand of S^T: lane (r, h) holds row r, dims 16s + 8h .. +7 for step s, rounded to f16 (q_f16);
    // rows of tokens past the block are zero
    const int tr = t0 + (r >> 3);
    half8 qb[16];
    {
        const float* qrow = q + ((size_t)min(tr, T - 1) * QH + kvh * GQA + (r & 7)) * HD + 8 * h;
#pragma unroll
        for (int s = 0; s < 16; s++) {
            float4 x0 = *(const float4*)(qrow + 16 * s), x1 = *(const float4*)(qrow + 16 * s + 4);
            if (tr >= T) x0 = x1 = make_float4(0.f, 0.f, 0.f, 0.f);
            qb[s] = half8{(_Float16)x0.x, (_Float16)x0.y, (_Float16)x0.z, (_Float16)x0.w,
                          (_Float16)x1.x, (_Float16)x1.y, (_Float16)x1.z, (_Float16)x1.w};
        }
    }
    const int vis = tr < T ? n + tr : 0;  // row r sees keys < vis
    const int kaddr = h * 512 + key_perm(r) * 16;
    float m = NEG_INF, lsum = 0.f;
    f32x16 O[8];
#pragma unroll
    for (int nb = 0; nb < 8; nb++) O[nb] = f32x16{};

    for (int j = 0; j < ntiles; j++) {
        wait_tiles(min(ntiles - 1 - j, NSLOT - 2));
        lds_barrier();  // tile j is in LDS for every wave; every wave is done with tile j - 1
        if (j + NSLOT - 1 < ntiles) issue(j + NSLOT - 1);
        const unsigned char* Ks = ring + (j % NSLOT) * SLOT_BYTES;
        const unsigned char* Vs = Ks + TILE_BYTES;
        const int k0 = cs + 32 * j;

        f32x16 S = f32x16{};
#pragma unroll
        for (int s = 0; s < 16; s++) S = mfma32(*(const half8*)(Ks + kaddr + s * 1024), qb[s], S);

        float mt = NEG_INF;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int key = k0 + 8 * h + i + (i >= 8 ? 8 : 0);
            const float sv = S[i] * scale2;
            S[i] = (key < vis && key >= start) ? sv : NEG_INF;
            mt = fmaxf(mt, S[i]);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        float mr = m;
        if (m == NEG_INF || mt > m + LAZY2) mr = fmaxf(m, mt);
        const float cf = (m == NEG_INF) ? 1.f : exp2f(m - mr);
        if (__any(cf != 1.f)) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float f = __shfl(cf, 8 * (i >> 2) + 4 * h + (i & 3));
#pragma unroll
                for (int nb = 0; nb < 8; nb++) O[nb][i] *= f;
            }
        }
        lsum *= cf;
        m = mr;
        half8 pa[2];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const _Float16 ph = (_Float16)(S[i] > NEG_INF ? exp2f(S[i] - mr) : 0.f);
            lsum += (float)ph;
            pa[i >> 3][i & 7] = ph;
        }
        const bool tail = k0 + 32 > kend;  // V rows past the written length may hold anything: keep 0 * V finite
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
            for (int nb = 0; nb < 8; nb++) {
                half8 vb = *(const half8*)(Vs + (2 * s2 + h) * 4096 + (32 * nb + r) * 16);
                if (tail) {
#pragma unroll
                    for (int jj = 0; jj < 8; jj++)
                        if (k0 + 16 * s2 + 8 * h + jj >= kend) vb[jj] = (_Float16)0.f;
                }
                O[nb] = mfma32(pa[s2], vb, O[nb]);
            }
    }
    lsum += __shfl_xor(lsum, 32);

    // partials of this wave's rows of present tokens: row index t*8 + head of the kv head, rows per kv head = 8T
    const size_t rpk = (size_t)T * GQA;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int ri = 8 * (i >> 2) + 4 * h + (i & 3);
        if (t0 + (ri >> 3) < T) {
            float* p = part + ((kvh * rpk + (size_t)t0 * GQA + ri) * nch + sp) * PART + PACC + r;
#pragma unroll
            for (int nb = 0; nb < 8; nb++) p[32 * nb] = O[nb][i];
        }
    }
    if (h == 0 && tr < T) {
        float* p = part + ((kvh * rpk + (size_t)t0 * GQA + r) * nch + sp) * PART;
        p[0] = m;
        p[1] = lsum;
    }
}

}  // namespace

PrefillPlan prefill_plan(int T, int n) {
    const int kend = n + T - 1;
    const int blocks = 2 * ((T + PT - 1) / PT);       // work-groups per split
    int nch = 256 / blocks;                           // about one work-group per CU
    nch = nch < 1 ? 1 : nch > 16 ? 16 : nch;
    int ch = (kend + nch - 1) / nch;
    ch = (ch + KBLK - 1) / KBLK * KBLK;               // whole 32-key tiles
    return PrefillPlan{ch, (kend + ch - 1) / ch};
}

size_t prefill_ws_floats(int T, int nch) { return (size_t)KVH * T * GQA * nch * PART; }

hipError_t launch_prefill(const Geom& g, const void* base, int layer, const float* q, int T, int n, int start,
                          float scale, const PrefillPlan& p, float* ws, const Launch& L) {
    if (g.fmt != 0) return hipErrorNotSupported;
    const char* b = (const char*)base;
    const void* kp = b + g.plane(layer, 0, 0) * g.plane_bytes();
    const void* vp = b + g.plane(layer, 1, 0) * g.plane_bytes();
    dim3 grid((T + PT - 1) / PT, p.nch, KVH);
    return launch(prefill_f16, grid, dim3(256), L, kp, vp, g.plane_elems, q, T, n, start, scale * LOG2E, p.ch, p.nch,
                  ws);
}

}  // namespace mkv
