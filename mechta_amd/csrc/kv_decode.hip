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
#include "mkv_internal.h"

namespace mkv {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LAZY2 = 8.0f * LOG2E;  // DM_LAZY = 8 (dmx.rs:124) in log2 units
constexpr float NEG_INF = -__builtin_huge_valf();

__device__ inline f32x16 mfma32(half8 a, half8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Key offset inside a 32-key tile of the K row loaded by A-operand row m. The C layout of the 32x32 MFMA gives lane
// half h the rows 8a + 4h + b (register 4a + b); loading row m from key perm(m) makes register i of lane half h hold
// key 8h + i (i < 8) or 16 + 8h + (i - 8) (i >= 8): exactly the keys the P operand of the PV MFMA needs in that lane.
__device__ inline int key_perm(int m) {
    int a = m >> 3, c = (m >> 2) & 1, b = m & 3;
    return 16 * (a >> 1) + 8 * c + 4 * (a & 1) + b;
}

__global__ void __launch_bounds__(256) decode_f16(const _Float16* __restrict__ kplane, const _Float16* __restrict__ vplane,
                                                  size_t plane_elems, const float* __restrict__ q, int ntok, int n,
                                                  int start, float scale2, int ch, int nch, int c0,
                                                  float* __restrict__ part) {
    const int kvh = blockIdx.y, c = c0 + blockIdx.x;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int h = lane >> 5, r = lane & 31;
    const int kend = n + ntok - 1;
    const int cs = c * ch, ce = min(cs + ch, kend);
    const _Float16* K = kplane + (size_t)kvh * plane_elems;
    const _Float16* V = vplane + (size_t)kvh * plane_elems;

    // Q as the B operand: lane (r, h) holds row r, dims 16s + 8h + 0..7 for step s, rounded to f16 (q_dmx).
    const int t = r >> 3;
    const int vis = n + t;  // row r sees keys < vis
    half8 qb[16];
    {
        const float* qrow = q + ((size_t)t * QH + kvh * GQA + (r & 7)) * HD + 8 * h;
#pragma unroll
        for (int s = 0; s < 16; s++) {
            float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
            if (t < ntok) {
                x0 = *(const float4*)(qrow + 16 * s);
                x1 = *(const float4*)(qrow + 16 * s + 4);
            }
            qb[s] = half8{(_Float16)x0.x, (_Float16)x0.y, (_Float16)x0.z, (_Float16)x0.w,
                          (_Float16)x1.x, (_Float16)x1.y, (_Float16)x1.z, (_Float16)x1.w};
        }
    }
    float m = NEG_INF, lsum = 0.f;
    f32x16 O[8];
#pragma unroll
    for (int nb = 0; nb < 8; nb++) O[nb] = f32x16{};

    const int pk = key_perm(r);
    const int ntiles = (ce - cs + 31) / 32;
    for (int ti = w; ti < ntiles; ti += 4) {
        const int k0 = cs + ti * 32;
        // K tile: A operand of step s = 16 bytes of key k0 + pk, dims 16s + 8h .. +7
        const _Float16* kb = K + (size_t)(k0 / KBLK) * (KBLK * HD) + h * (KBLK * 8) + pk * 8;
        half8 ka[16];
#pragma unroll
        for (int s = 0; s < 16; s++) ka[s] = *(const half8*)(kb + s * 2 * (KBLK * 8));
        // V tile: B operand (dims 32nb + r, keys 16s2 + 8h .. +7) = 16 bytes of group k0/8 + 2s2 + h at dim
        const _Float16* vb = V + (size_t)(k0 / VGRP + h) * (VGRP * HD) + r * VGRP;
        half8 va[2][8];
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
            for (int nb = 0; nb < 8; nb++) va[s2][nb] = *(const half8*)(vb + s2 * 2 * (VGRP * HD) + nb * 32 * VGRP);

        f32x16 S = f32x16{};
#pragma unroll
        for (int s = 0; s < 16; s++) S = mfma32(ka[s], qb[s], S);

        float mt = NEG_INF;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            int key = k0 + 8 * h + i + (i >= 8 ? 8 : 0);
            float sv = S[i] * scale2;
            sv = (key < vis && key >= start) ? sv : NEG_INF;
            S[i] = sv;
            mt = fmaxf(mt, sv);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        float mr = m;
        if (m == NEG_INF || mt > m + LAZY2) mr = fmaxf(m, mt);
        float cf = (m == NEG_INF) ? 1.f : exp2f(m - mr);
        if (__any(cf != 1.f)) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                float f = __shfl(cf, 8 * (i >> 2) + 4 * h + (i & 3));
#pragma unroll
                for (int nb = 0; nb < 8; nb++) O[nb][i] *= f;
            }
        }
        lsum *= cf;
        m = mr;
        half8 pa[2];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            float p = S[i] > NEG_INF ? exp2f(S[i] - mr) : 0.f;
            _Float16 ph = (_Float16)p;
            lsum += (float)ph;
            pa[i >> 3][i & 7] = ph;
        }
        if (k0 + 32 > kend) {  // tail tile: V rows past the written length may hold anything; keep 0 * V finite
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
                for (int j = 0; j < 8; j++)
                    if (k0 + 16 * s2 + 8 * h + j >= kend)
#pragma unroll
                        for (int nb = 0; nb < 8; nb++) va[s2][nb][j] = (_Float16)0.f;
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
            for (int nb = 0; nb < 8; nb++) O[nb] = mfma32(pa[s2], va[s2][nb], O[nb]);
    }
    lsum += __shfl_xor(lsum, 32);

    // merge the 4 waves
    __shared__ float sm_m[4][32], sm_l[4][32];
    __shared__ float so[32][HD + 4];
    if (h == 0) {
        sm_m[w][r] = m;
        sm_l[w][r] = lsum;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) {
        int ri = 8 * (i >> 2) + 4 * h + (i & 3);
        float M = fmaxf(fmaxf(sm_m[0][ri], sm_m[1][ri]), fmaxf(sm_m[2][ri], sm_m[3][ri]));
        float mw = sm_m[w][ri];
        float f = mw == NEG_INF ? 0.f : exp2f(mw - M);
#pragma unroll
        for (int nb = 0; nb < 8; nb++) O[nb][i] *= f;
    }
    for (int ww = 0; ww < 4; ww++) {
        if (w == ww) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                int ri = 8 * (i >> 2) + 4 * h + (i & 3);
#pragma unroll
                for (int nb = 0; nb < 8; nb++) {
                    float* dst = &so[ri][32 * nb + r];
                    *dst = ww == 0 ? O[nb][i] : *dst + O[nb][i];
                }
            }
        }
        __syncthreads();
    }
    const int nrows = 8 * ntok;
    for (int row = 0; row < nrows; row++) {
        float* p = part + ((size_t)(kvh * ROWS + row) * nch + c) * PART;
        p[2 + threadIdx.x] = so[row][threadIdx.x];
    }
    if (threadIdx.x < nrows) {
        int row = threadIdx.x;
        float M = fmaxf(fmaxf(sm_m[0][row], sm_m[1][row]), fmaxf(sm_m[2][row], sm_m[3][row]));
        float L = 0.f;
        for (int ww = 0; ww < 4; ww++)
            if (sm_m[ww][row] != NEG_INF) L += exp2f(sm_m[ww][row] - M) * sm_l[ww][row];
        float* p = part + ((size_t)(kvh * ROWS + row) * nch + c) * PART;
        p[0] = M;
        p[1] = L;
    }
}

// f32 store: VALU flash decode, 32-key tiles staged in LDS; thread (row, 4 keys) for S, thread = dim for P.V.
__global__ void __launch_bounds__(256) decode_f32(const float* __restrict__ kplane, const float* __restrict__ vplane,
                                                  size_t plane_elems, const float* __restrict__ q, int ntok, int n,
                                                  int start, float scale2, int ch, int nch, int c0,
                                                  float* __restrict__ part) {
    const int kvh = blockIdx.y, c = c0 + blockIdx.x, tid = threadIdx.x;
    const int kend = n + ntok - 1;
    const int cs = c * ch, ce = min(cs + ch, kend);
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
        p[2 + tid] = acc[row];
        if (tid == 0) {
            p[0] = sm_m[row];
            p[1] = sm_l[row];
        }
    }
}

__global__ void __launch_bounds__(256) decode_combine(const float* __restrict__ part, int n, int start, int ch,
                                                      int nch, const float* __restrict__ gate,
                                                      float* __restrict__ out) {
    const int t = blockIdx.x / QH, head = blockIdx.x % QH, d = threadIdx.x;
    const int kvh = head / GQA, row = t * GQA + head % GQA;
    const float* p = part + (size_t)(kvh * ROWS + row) * nch * PART;
    const int c0 = start / ch, c1 = (n + t + ch - 1) / ch;  // chunks holding a key of [start, n + t)
    float M = NEG_INF;
    for (int c = c0; c < c1; c++) M = fmaxf(M, p[(size_t)c * PART]);
    float L = 0.f, acc = 0.f;
    for (int c = c0; c < c1; c++) {
        const float* pc = p + (size_t)c * PART;
        float mc = pc[0];
        if (mc == NEG_INF) continue;
        float e = exp2f(mc - M);
        L += e * pc[1];
        acc += e * pc[2 + d];
    }
    float o = acc / L;
    if (gate) {
        float g = gate[((size_t)t * QH + head) * 512 + 256 + d];
        o = o * (1.f / (1.f + expf(-g)));
    }
    out[((size_t)t * QH + head) * HD + d] = o;
}

}  // namespace

DecodePlan decode_plan(int n, int ntok, int start) {
    const int kend = n + ntok - 1;
    int ch = (kend + 127) / 128;  // about 128 chunks per kv head: 256 work-groups for 256 CUs
    ch = (ch + 31) / 32 * 32;     // whole 32-key tiles
    if (ch < 128) ch = 128;
    return DecodePlan{ch, (kend + ch - 1) / ch, start / ch};
}

hipError_t launch_decode_core(const Geom& g, const void* base, int layer, const float* q, int ntok, int n, int start,
                              float scale, const DecodePlan& p, const DecodeWs& ws, hipStream_t s) {
    if (p.nch > ws.max_chunks) return hipErrorInvalidValue;
    const char* b = (const char*)base;
    const void* kp = b + g.plane(layer, 0, 0) * g.plane_bytes();
    const void* vp = b + g.plane(layer, 1, 0) * g.plane_bytes();
    const float scale2 = scale * LOG2E;
    dim3 grid(p.nch - p.c0, KVH);
    if (g.fmt == 0)
        decode_f16<<<grid, 256, 0, s>>>((const _Float16*)kp, (const _Float16*)vp, g.plane_elems, q, ntok, n, start,
                                        scale2, p.ch, p.nch, p.c0, ws.part);
    else
        decode_f32<<<grid, 256, 0, s>>>((const float*)kp, (const float*)vp, g.plane_elems, q, ntok, n, start, scale2,
                                        p.ch, p.nch, p.c0, ws.part);
    return hipGetLastError();
}

hipError_t launch_decode_merge(int ntok, int n, int start, const DecodePlan& p, const DecodeWs& ws, const float* gate,
                               float* out, hipStream_t s) {
    decode_combine<<<ntok * QH, 256, 0, s>>>(ws.part, n, start, p.ch, p.nch, gate, out);
    return hipGetLastError();
}

}  // namespace mkv
