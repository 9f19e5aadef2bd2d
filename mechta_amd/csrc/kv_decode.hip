// kv_decode.hip -- split-K flash decode for 1..4 query tokens (GQA 8:1) and the merge of the partials.
//
// Replaces attn_fd (ops.wgsl:310-394), q_dmx + attn_dmx2 (dmx.rs:19-138) and attn_fd_combine (ops.wgsl:523-538).
//
// f16 store (decode_f16): a work-group = (chunk of `ch` positions, kv head); its 4 waves take the chunk's 32-key
// tiles round robin. The 8 query heads of the kv head times the ntok tokens are 32 query rows (row = t*8 + head,
// rows of absent tokens are zero), so one wave does, per tile:
//   S^T[32 keys][32 rows] = K_tile . Q^T   16 x v_mfma_f32_32x32x16_f16 (A = K straight from the tiled plane)
//   online softmax of the 32 rows, lazy reference max (moves when first or when the tile max exceeds it by > 8,
//   as attn_dmx, dmx.rs:72-74), P rounded to f16, l += f32(P)
//   O[32 rows][256] += P . V_tile           16 x v_mfma_f32_32x32x16_f16 (B = V straight from the grouped plane)
// K and V tiles are read once per work-group with 16-byte loads, each load instruction covering 2 x 512 contiguous
// bytes, so the kernel is a coalesced HBM stream; the tile's 32 KB are in flight before the first MFMA.
// The 4 waves' (m, l, O) are merged in LDS and the work-group writes one partial [m, l, acc[256]] per row.
//
// f32 store (decode_f32): same grid and partials, f32 VALU math with K, V and Q staged through LDS.
//
// decode_combine: one work-group per (token, head), thread = dim: o = sum_c 2^(m_c - M) acc_c / sum_c 2^(m_c - M) l_c
// over the chunks holding a visible key, then the optional sigmoid output gate (attn_gate, ops.wgsl:171-177).
// Partials keep m in log2 units (scores are pre-multiplied by scale * log2 e).
#include <type_traits>

#include "mkv_device.h"

namespace mkv {
namespace {

constexpr int KPS = 64;                        // keys per stage of the decode ring
constexpr int PS_STRIDE = KPS + 8;             // halves per P row in LDS (conflict-free 16-byte reads)
constexpr int MERGE_FEW = 16;  // chunks of the one-lane-per-dim merge
constexpr int MERGE_J = 9;  // chunks per merge lane: 16 lanes x 9 >= the at most 130 chunks of decode_plan

// One stage of this wave's registers: K operands (16 keys x 128 dims) and V operands (64 keys x 32 dims).
struct StageRegs {
    half8 k[4];
    half8 v[4];
};

__global__ void __launch_bounds__(512) decode_f16(_Float16* __restrict__ kplane, _Float16* __restrict__ vplane,
                                                  size_t plane_elems, const float* __restrict__ q, int ntok, int n,
                                                  int start, float scale2, int span, int nch, int c0,
                                                  float* __restrict__ part, const float* __restrict__ akn,
                                                  const float* __restrict__ av, const float* __restrict__ atab,
                                                  int apos, int antok) {
    const int kvh = blockIdx.y, c = c0 + blockIdx.x, tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int h = lane >> 5, r = lane & 31, l16 = lane & 15, g4 = lane >> 4;
    const int kend = n + ntok - 1;
    const int cs = chunk_lo(c, span, nch), ce = c + 1 < nch ? chunk_lo(c + 1, span, nch) : kend;
    _Float16* K = kplane + (size_t)kvh * plane_elems;
    _Float16* V = vplane + (size_t)kvh * plane_elems;

    __shared__ __attribute__((aligned(16))) float ss[2][ROWS][KPS + 4];  // partial S of the two dim halves [row][key]
    __shared__ __attribute__((aligned(16))) _Float16 ps[ROWS][PS_STRIDE];
    __shared__ __attribute__((aligned(16))) float cfs[ROWS];

    // Fused append (mkv_append_decode): the work-group whose chunk holds new rows writes this kv head's K and V of
    // those rows (the same arithmetic as append_kernel) and makes them visible before any stage is loaded.
    {
        const int p0 = max(apos, cs), p1 = min(apos + antok, ce);
        if (p0 < p1) {
            unsigned short* Ku = (unsigned short*)K;
            unsigned short* Vu = (unsigned short*)V;
            for (int it = tid; it < (p1 - p0) * 32; it += 512) {
                const int p = p0 + (it >> 5), d0 = (it & 31) * 8, t = p - apos;
                const float* a = akn + ((size_t)t * KVH + kvh) * HD;
                const float* tb = atab + (size_t)t * 64;
                u16x8 w8;
#pragma unroll
                for (int j = 0; j < 8; j++) w8[j] = f2h(rope_dim(a, tb, d0 + j));
                *(u16x8*)(Ku + k_off(p, d0)) = w8;
            }
            for (int it = tid; it < (p1 - p0) * HD; it += 512) {
                const int p = p0 + it / HD, d = it % HD;
                Vu[v_off(p, d)] = f2h(av[(size_t)(p - apos) * (KVH * HD) + kvh * HD + d]);
            }
            __threadfence();
            __syncthreads();
        }
    }

    // Roles of wave w in a 64-key stage:
    //   S: keys 16kq .. 16kq + 15 (kq = w % 4) times dims 128dh .. 128dh + 127 (dh = w / 4), both 16-row halves,
    //      v_mfma_f32_16x16x32_f16 with A = K (lane: key 16kq + lane%16, 8 dims at 32s + 8(lane/16)), B = Q^T;
    //      the two dim halves' partial S meet in LDS;
    //   P.V: dims 32w .. 32w + 31 of all 32 rows, v_mfma_f32_32x32x16_f16, B = V (lane: dim 32w + lane%32,
    //      8 keys 16s2 + 8(lane/32) .. of group 2s2 + lane/32).
    const int kq = w & 3, dh = w >> 2;
    const int nst = (ce - cs + KPS - 1) / KPS;
    const int kkey = 16 * kq + l16;  // S-role key inside the stage
    auto load = [&](int j, StageRegs& R) {
        const int k0 = cs + j * KPS;
        const _Float16* kb = K + (size_t)((k0 + kkey) / KBLK) * (KBLK * HD) + ((k0 + kkey) % KBLK) * 8;
#pragma unroll
        for (int s = 0; s < 4; s++) R.k[s] = *(const half8*)(kb + (16 * dh + 4 * s + g4) * (KBLK * 8));
        const _Float16* vb = V + (size_t)(k0 / VGRP + h) * (VGRP * HD) + (32 * w + r) * VGRP;
#pragma unroll
        for (int s2 = 0; s2 < 4; s2++) R.v[s2] = *(const half8*)(vb + s2 * 2 * (VGRP * HD));
    };
    StageRegs RA, RB, RC;
    if (nst > 0) load(0, RA);
    if (nst > 1) load(1, RB);

    // Q (rounded to f16 as q_dmx) as B operand, straight into registers: rows 16hb + lane%16, dims
    // 128dh + 32s + 8(lane/16) .. +7; rows of absent tokens are zero
    half8 qb[2][4];
#pragma unroll
    for (int hb = 0; hb < 2; hb++) {
        const int row = 16 * hb + l16, tq = row >> 3;
        const float* qr = q + ((size_t)min(tq, ntok - 1) * QH + kvh * GQA + (row & 7)) * HD + 128 * dh + 8 * g4;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            float4 x0 = *(const float4*)(qr + 32 * s), x1 = *(const float4*)(qr + 32 * s + 4);
            if (tq >= ntok) x0 = x1 = make_float4(0.f, 0.f, 0.f, 0.f);
            qb[hb][s] = half8{(_Float16)x0.x, (_Float16)x0.y, (_Float16)x0.z, (_Float16)x0.w,
                              (_Float16)x1.x, (_Float16)x1.y, (_Float16)x1.z, (_Float16)x1.w};
        }
    }

    // softmax role: thread (srow, sq) owns keys 4sq .. 4sq+3 of row srow; the row's 16 threads keep identical m, l
    const int srow = tid >> 4, sq = tid & 15;
    const int vis = n + (srow >> 3);  // row srow sees keys < vis
    float m_run = NEG_INF, l_run = 0.f;
    f32x16 O = f32x16{};

    auto stage = [&](int j, StageRegs& R, StageRegs& Rnext2, auto steady) {
        // two stages in flight while this one is computed (unconditional in the steady loop: branches around loads
        // make the compiler's wait counts pessimistic)
        if (decltype(steady)::value || j + 2 < nst) load(j + 2, Rnext2);
        const int k0 = cs + j * KPS;
        f32x4 s4[2] = {f32x4{}, f32x4{}};
#pragma unroll
        for (int s = 0; s < 4; s++) {
            s4[0] = mfma16(R.k[s], qb[0][s], s4[0]);
            s4[1] = mfma16(R.k[s], qb[1][s], s4[1]);
        }
#pragma unroll
        for (int hb = 0; hb < 2; hb++)
#pragma unroll
            for (int i = 0; i < 4; i++) ss[dh][16 * hb + l16][16 * kq + 4 * g4 + i] = s4[hb][i];
        lds_barrier();

        // online softmax with the lazy reference max of attn_dmx (dmx.rs:72-86), log2 units
        const float4 x0 = *(const float4*)&ss[0][srow][4 * sq];
        const float4 x1 = *(const float4*)&ss[1][srow][4 * sq];
        float sv[4] = {(x0.x + x1.x) * scale2, (x0.y + x1.y) * scale2, (x0.z + x1.z) * scale2, (x0.w + x1.w) * scale2};
        if (!(k0 >= start && k0 + KPS <= min(n, ce))) {  // the stage crosses a row's window or the chunk end
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = k0 + 4 * sq + i;
                if (!(key < vis && key >= start && key < ce)) sv[i] = NEG_INF;
            }
        }
        float mt = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        mt = reduce16(mt, [](float a, float b) { return fmaxf(a, b); });
        float mr = m_run;
        if (m_run == NEG_INF || mt > m_run + LAZY2) mr = fmaxf(m_run, mt);
        const float cf = m_run == NEG_INF ? 1.f : fast_exp2(m_run - mr);
        const float base = mr == NEG_INF ? 0.f : mr;  // masked scores are -inf: 2^-inf = 0
        float psum = 0.f;
        _Float16 p4[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            p4[i] = (_Float16)fast_exp2(sv[i] - base);
            psum += (float)p4[i];
        }
        *(uint2*)&ps[srow][4 * sq] = *(const uint2*)p4;
        psum = reduce16(psum, [](float a, float b) { return a + b; });
        l_run = l_run * cf + psum;
        m_run = mr;
        if (sq == 0) cfs[srow] = cf;
        lds_barrier();

        if (__any(cfs[r] != 1.f)) {
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const float4 f = *(const float4*)&cfs[8 * a + 4 * h];
                O[4 * a] *= f.x;
                O[4 * a + 1] *= f.y;
                O[4 * a + 2] *= f.z;
                O[4 * a + 3] *= f.w;
            }
        }
        const bool tail = k0 + KPS > kend;  // V rows past the written length may hold anything: keep 0 * V finite
#pragma unroll
        for (int s2 = 0; s2 < KPS / 16; s2++) {
            const half8 pa = *(const half8*)&ps[r][16 * s2 + 8 * h];
            half8 vb = R.v[s2];
            if (tail) {
#pragma unroll
                for (int jj = 0; jj < 8; jj++)
                    if (k0 + 16 * s2 + 8 * h + jj >= kend) vb[jj] = (_Float16)0.f;
            }
            O = mfma32(pa, vb, O);
        }
    };
    // register sets rotate with period 3: (this stage, stage + 2) = (A, C), (B, A), (C, B)
    int j = 0;
    for (; j + 5 <= nst; j += 3) {
        stage(j, RA, RC, std::true_type{});
        stage(j + 1, RB, RA, std::true_type{});
        stage(j + 2, RC, RB, std::true_type{});
    }
    if (j < nst) stage(j, RA, RC, std::false_type{});
    if (j + 1 < nst) stage(j + 1, RB, RA, std::false_type{});
    if (j + 2 < nst) stage(j + 2, RC, RB, std::false_type{});
    if (j + 3 < nst) stage(j + 3, RA, RC, std::false_type{});

    // partials: this wave's 32 dims of every row of a present token; m and l from the rows' softmax threads
    const int nrows = 8 * ntok;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int ri = 8 * (i >> 2) + 4 * h + (i & 3);
        if (ri < nrows) part[((size_t)(kvh * ROWS + ri) * nch + c) * PART + PACC + 32 * w + r] = O[i];
    }
    if (sq == 0 && srow < nrows) {
        float* p = part + ((size_t)(kvh * ROWS + srow) * nch + c) * PART;
        p[0] = m_run;
        p[1] = l_run;
    }
}

// f32 store: VALU flash decode, 32-key tiles staged in LDS; thread (row, 4 keys) for S, thread = dim for P.V.
__global__ void __launch_bounds__(256) decode_f32(const float* __restrict__ kplane, const float* __restrict__ vplane,
                                                  size_t plane_elems, const float* __restrict__ q, int ntok, int n,
                                                  int start, float scale2, int span, int nch, int c0,
                                                  float* __restrict__ part) {
    const int kvh = blockIdx.y, c = c0 + blockIdx.x, tid = threadIdx.x;
    const int kend = n + ntok - 1;
    const int cs = chunk_lo(c, span, nch), ce = c + 1 < nch ? chunk_lo(c + 1, span, nch) : kend;
    const float* K = kplane + (size_t)kvh * plane_elems;
    const float* V = vplane + (size_t)kvh * plane_elems;
    const int nrows = 8 * ntok;
    __shared__ float qs[ROWS][HD + 1];
    __shared__ float kv[32][HD + 1];
    __shared__ float ps[ROWS][33];
    __shared__ float sm_m[ROWS], sm_l[ROWS], sm_c[ROWS];
    for (int i = tid; i < ROWS * HD; i += 256) {
        int row = i / HD, d = i % HD;
        int t = row >> 3;
        qs[row][d] = t < ntok ? q[((size_t)t * QH + kvh * GQA + (row & 7)) * HD + d] : 0.f;
    }
    if (tid < ROWS) {
        sm_m[tid] = NEG_INF;
        sm_l[tid] = 0.f;
    }
    float acc[ROWS];
#pragma unroll
    for (int i = 0; i < ROWS; i++) acc[i] = 0.f;
    const int srow = tid >> 3, sq = tid & 7;  // S: row srow, keys 4sq .. 4sq+3
    for (int k0 = cs; k0 < ce; k0 += 32) {
        __syncthreads();
        for (int i = tid; i < 32 * HD / 4; i += 256) {
            int key = i / (HD / 4), d4 = (i % (HD / 4)) * 4;
            float4 x = *(const float4*)(K + (size_t)(k0 + key) * HD + d4);
            kv[key][d4] = x.x; kv[key][d4 + 1] = x.y; kv[key][d4 + 2] = x.z; kv[key][d4 + 3] = x.w;
        }
        __syncthreads();
        float s4[4] = {0.f, 0.f, 0.f, 0.f};
        for (int d = 0; d < HD; d++) {
            float qv = qs[srow][d];
#pragma unroll
            for (int j = 0; j < 4; j++) s4[j] += qv * kv[4 * sq + j][d];
        }
        const int vis = n + (srow >> 3);
        float mt = NEG_INF;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int key = k0 + 4 * sq + j;
            s4[j] = (key < vis && key >= start && key < ce) ? s4[j] * scale2 : NEG_INF;
            mt = fmaxf(mt, s4[j]);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 1));
        mt = fmaxf(mt, __shfl_xor(mt, 2));
        mt = fmaxf(mt, __shfl_xor(mt, 4));
        float mo = sm_m[srow];
        float mx = fmaxf(mo, mt);
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float p = s4[j] > NEG_INF ? exp2f(s4[j] - mx) : 0.f;
            ps[srow][4 * sq + j] = p;
            sum += p;
        }
        sum += __shfl_xor(sum, 1);
        sum += __shfl_xor(sum, 2);
        sum += __shfl_xor(sum, 4);
        __syncthreads();  // everyone has read sm_m[srow] and K
        if (sq == 0) {
            float cf = mo == NEG_INF ? 0.f : exp2f(mo - mx);
            sm_c[srow] = cf;
            sm_m[srow] = mx;
            sm_l[srow] = sm_l[srow] * cf + sum;
        }
        for (int i = tid; i < 32 * HD / 4; i += 256) {
            int key = i / (HD / 4), d4 = (i % (HD / 4)) * 4;
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k0 + key < kend) x = *(const float4*)(V + (size_t)(k0 + key) * HD + d4);
            kv[key][d4] = x.x; kv[key][d4 + 1] = x.y; kv[key][d4 + 2] = x.z; kv[key][d4 + 3] = x.w;
        }
        __syncthreads();
#pragma unroll
        for (int row = 0; row < ROWS; row++) acc[row] *= sm_c[row];
        for (int j = 0; j < 32; j++) {
            float v = kv[j][tid];
#pragma unroll
            for (int row = 0; row < ROWS; row++) acc[row] += ps[row][j] * v;
        }
    }
    __syncthreads();
    for (int row = 0; row < nrows; row++) {
        float* p = part + ((size_t)(kvh * ROWS + row) * nch + c) * PART;
        p[PACC + tid] = acc[row];
        if (tid == 0) {
            p[0] = sm_m[row];
            p[1] = sm_l[row];
        }
    }
}

// Merge of the split-K partials: work-group (token, head, quarter of the dims); its 256 threads are 16 chunk lanes x
// 16 dim lanes (4 dims each), so every chunk's 64 dims are one coalesced 256-byte read and all chunks are in flight at
// once; the 16 chunk lanes are then summed in LDS.
__global__ void __launch_bounds__(256) decode_combine(const float* __restrict__ part, int rpk, int n, int start,
                                                      int span, int nch, const float* __restrict__ gate,
                                                      float* __restrict__ out) {
    const int t = blockIdx.x / QH, head = blockIdx.x % QH, dq = blockIdx.y, tid = threadIdx.x;
    const int kvh = head / GQA, row = t * GQA + head % GQA;
    const float* p = part + ((size_t)kvh * rpk + row) * nch * PART;
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
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
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
        const int dd = tid >> 2, comp = tid & 3;
        float sum = 0.f, lt = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float4 v = acc4[i][dd];
            sum += comp == 0 ? v.x : comp == 1 ? v.y : comp == 2 ? v.z : v.w;
            lt += redl[i];
        }
        const int d = dq * 64 + tid;
        float o = sum / lt;
        if (gate) {
            const float g = gate[((size_t)t * QH + head) * 512 + 256 + d];
            o = o * (1.f / (1.f + expf(-g)));
        }
        out[((size_t)t * QH + head) * HD + d] = o;
    }
}

// Merge for few chunks (prefill splits): work-group = (token, head), thread = dim; all chunks of the row are loaded
// in one round trip.
__global__ void __launch_bounds__(256) merge_few(const float* __restrict__ part, int rpk, int n, int start, int span,
                                                 int nch, const float* __restrict__ gate, float* __restrict__ out) {
    const int t = blockIdx.x / QH, head = blockIdx.x % QH, d = threadIdx.x;
    const int kvh = head / GQA, row = t * GQA + head % GQA;
    const float* p = part + ((size_t)kvh * rpk + row) * nch * PART;
    int c0, c1;  // chunks holding a key of [start, n + t)
    chunk_range(start, n + t, span, nch, c0, c1);
    float mj[MERGE_FEW], lj[MERGE_FEW], aj[MERGE_FEW];
    float M = NEG_INF;
#pragma unroll
    for (int j = 0; j < MERGE_FEW; j++) {
        const int c = c0 + j;
        mj[j] = NEG_INF;
        lj[j] = aj[j] = 0.f;
        if (c < c1) {
            const float* pc = p + (size_t)c * PART;
            mj[j] = pc[0];
            lj[j] = pc[1];
            aj[j] = pc[PACC + d];
        }
        M = fmaxf(M, mj[j]);
    }
    float L = 0.f, acc = 0.f;
#pragma unroll
    for (int j = 0; j < MERGE_FEW; j++) {
        const float e = mj[j] == NEG_INF ? 0.f : exp2f(mj[j] - M);
        L += e * lj[j];
        acc += e * aj[j];
    }
    float o = acc / L;
    if (gate) {
        const float g = gate[((size_t)t * QH + head) * 512 + 256 + d];
        o = o * (1.f / (1.f + expf(-g)));
    }
    out[((size_t)t * QH + head) * HD + d] = o;
}

}  // namespace

DecodePlan decode_plan(int n, int ntok, int start) {
    const int kend = n + ntok - 1;
    // chunks of at least 128 positions, at most 124 per kv head: 248 work-groups on the 256 CUs, one each. (Measured
    // at 64K positions: 124 chunks of 512 or 544 positions beat 128, 120 and 112 -- the work-group with the most
    // 64-position stages sets the time.)
    int nch = kend / 128;
    nch = nch < 1 ? 1 : nch > 124 ? 124 : nch;
    // boundaries planned over kend + half a chunk: the last chunk, whose work-group also writes the appended rows
    // (mkv_append_decode), is about half as long as the others and does not finish last
    const int span = kend + kend / (2 * nch);
    int c0, c1;
    chunk_range(start, kend, span, nch, c0, c1);
    return DecodePlan{span, nch, c0};
}

hipError_t launch_decode_core(const Geom& g, void* base, int layer, const float* q, int ntok, int n, int start,
                              float scale, const DecodePlan& p, const DecodeWs& ws, const FusedAppend& fa,
                              const Launch& L) {
    if (p.nch > ws.max_chunks || p.nch - p.c0 > 16 * MERGE_J) return hipErrorInvalidValue;
    char* b = (char*)base;
    void* kp = b + g.plane(layer, 0, 0) * g.plane_bytes();
    void* vp = b + g.plane(layer, 1, 0) * g.plane_bytes();
    const float scale2 = scale * LOG2E;
    dim3 grid(p.nch - p.c0, KVH);
    if (g.fmt == 0)
        return launch(decode_f16, grid, dim3(512), L, kp, vp, g.plane_elems, q, ntok, n, start, scale2, p.span, p.nch,
                      p.c0, ws.part, fa.kn, fa.v, fa.tab, fa.pos, fa.ntok);
    if (fa.ntok) return hipErrorNotSupported;
    return launch(decode_f32, grid, dim3(256), L, kp, vp, g.plane_elems, q, ntok, n, start, scale2, p.span, p.nch, p.c0,
                  ws.part);
}

hipError_t launch_merge(const float* part, int rpk, int ntok, int n, int start, int span, int nch, const float* gate,
                        float* out, const Launch& L) {
    if (nch > 16 * MERGE_J) return hipErrorInvalidValue;
    if (nch <= MERGE_FEW)
        return launch(merge_few, dim3(ntok * QH), dim3(256), L, part, rpk, n, start, span, nch, gate, out);
    return launch(decode_combine, dim3(ntok * QH, HD / 64), dim3(256), L, part, rpk, n, start, span, nch, gate, out);
}

hipError_t launch_decode_merge(int ntok, int n, int start, const DecodePlan& p, const DecodeWs& ws, const float* gate,
                               float* out, const Launch& L) {
    return launch_merge(ws.part, ROWS, ntok, n, start, p.span, p.nch, gate, out, L);
}

}  // namespace mkv
