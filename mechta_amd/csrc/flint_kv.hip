// flint_kv.hip -- the Flint model's KV path: ring append, NEOX RoPE, conversion to the reference's row layout, and
// sliding-window attention with per-head sinks (flint_attn.wgsl:1-257), for one decode token or a prefill block.
//
// Attention work-group: (block of 4 tokens, key split, kv head) = 32 query rows (token * 8 + head) against the split's
// keys in tiles of 32 positions, on the fp32 matrix cores (v_mfma_f32_32x32x2_f32; f16 caches are widened on load,
// the arithmetic is f32 as the reference's). Per tile, wave w of a group of 4:
//   S^T[32 keys][32 rows] over dims 32w .. 32w+31    16 MFMAs, A = K straight from HBM, B = Q (LDS)
//   the four partial S^T summed through LDS in one order, exact-max online softmax (redundantly in every wave)
//   O[32 rows][dims 32w .. 32w+31] += P . V           16 MFMAs, A = P (the S^T registers), B = V
// The 32x32 accumulator layout gives lane l (half s = l / 32) row l % 32 and keys 8a + 4s + b (register 4a + b), the
// keys the A operand of the P.V MFMAs needs in that lane; with V stored in groups of 4 (f32) or 8 (f16) positions each
// register quad's operand is one 16-byte (f32) or 8-byte (f16) load. Rows are positions modulo the ring: a 32-position
// tile is one 32-row block (rings are multiples of 32), so a ring wrap only changes the tile's base address.
// Each split writes one partial [m, l, 0, 0, acc[128]] per row; fl_merge adds the sink (as attn_fd_merge,
// flint_attn.wgsl:241-257: the sink joins the maximum and the sum, never the output) and normalizes.
#include "flint_internal.h"
#include "mkv_device.h"

namespace mkv {
namespace flint {
namespace {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));

constexpr int TILE = 32;
constexpr int QPAD = HD + 4;  // LDS row of Q (floats)

__device__ inline f32x16 mfma32f(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Window start of the token at position p: the 513 positions up to p on sliding layers (lo_di, flint_attn.wgsl:84).
__device__ inline int window_lo(int p, int win) { return win > 0 && p + 1 > win ? p + 1 - win : 0; }

template <int FMT>
struct TileRegs;
template <>
struct TileRegs<1> {  // f32: K dims 32w + 8m + 4s .. +3 of key l % 32 (m < 4); V keys 8q + 4s .. +3 of dim 32w + l % 32
    f32x4 k[4];
    f32x4 v[4];
};
template <>
struct TileRegs<0> {  // f16: K dims 32w + 16a + 8s .. +7 (a < 2); V as f32, 4 halves
    half8 k[2];
    half4 v[4];
};

template <int FMT, int NWG>
__global__ void __launch_bounds__(256 * NWG) fl_attn(const void* __restrict__ kplane, const void* __restrict__ vplane,
                                                     size_t plane_elems, int rows, const float* __restrict__ q, int T,
                                                     int pos0, int win, float scale2, int klo, int span, int nch,
                                                     int nrb, float* __restrict__ part) {
    constexpr int BPE = FMT == 1 ? 4 : 2;
    constexpr unsigned TILE_BYTES = TILE * HD * BPE;
    const int G = gridDim.x, L = blockIdx.x;
    const int W = G % NXCD == 0 ? (L % NXCD) * (G / NXCD) + L / NXCD : L;
    const int rb = W % nrb, c = (W / nrb) % nch, kvh = W / nrb / nch;
    const int tid = threadIdx.x, lane = tid & 63, grp = tid >> 8, w = (tid >> 6) & 3, s = lane >> 5, r32 = lane & 31;
    const int t0 = 4 * rb, nt = min(4, T - t0);
    const int lo_first = window_lo(pos0 + t0, win);  // the block's earliest visible position
    const int cs = klo + chunk_lo(c, span, nch), ce = c + 1 < nch ? klo + chunk_lo(c + 1, span, nch) : klo + span;
    const int lo = max(cs, lo_first / TILE * TILE), hi = min(ce, pos0 + t0 + nt);  // keys [lo, hi) of this split
    const int ntile = hi > lo ? (hi - lo + TILE - 1) / TILE : 0;

    __shared__ float qs[32][QPAD];
    __shared__ f32x4 sx[2][NWG][4][4][64];  // partial S^T: [round parity][group][wave][register quad][lane]
    for (int i = tid; i < 32 * HD / 4; i += 256 * NWG) {
        const int row = i / (HD / 4), d4 = (i % (HD / 4)) * 4, t = t0 + (row >> 3);
        f32x4 x = f32x4{};
        if (t < T) x = *(const f32x4*)(q + ((size_t)t * QH + kvh * GQA + (row & 7)) * HD + d4);
        *(f32x4*)&qs[row][d4] = x;
    }
    __syncthreads();

    // the whole plane is the resource; tiles past the last start at the plane's end, so all their loads lie past it
    // (zeros, no memory access)
    const unsigned pbytes = (unsigned)(plane_elems * BPE);
    const rsrc_t kr = plane_rsrc((const char*)kplane + (size_t)kvh * plane_elems * BPE, pbytes);
    const rsrc_t vr = plane_rsrc((const char*)vplane + (size_t)kvh * plane_elems * BPE, pbytes);
    auto tile_base = [&](int j) -> unsigned {
        return j < ntile ? (unsigned)((lo + j * TILE) % rows) * (HD * BPE) : pbytes;
    };
    auto load = [&](TileRegs<FMT>& X, int j) {
        const unsigned b = tile_base(j);
        if constexpr (FMT == 1) {
#pragma unroll
            for (int m = 0; m < 4; m++)
                X.k[m] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                       kr, b + ((8 * w + 2 * m + s) * TILE + r32) * 16, 0, 0));
#pragma unroll
            for (int qq = 0; qq < 4; qq++)
                X.v[qq] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        vr, b + ((2 * qq + s) * HD + 32 * w + r32) * 16, 0, 0));
        } else {
#pragma unroll
            for (int a = 0; a < 2; a++)
                X.k[a] = bload16(kr, b + ((4 * w + 2 * a + s) * TILE + r32) * 16);
#pragma unroll
            for (int qq = 0; qq < 4; qq++)
                X.v[qq] = __builtin_bit_cast(half4, __builtin_amdgcn_raw_buffer_load_b64(
                                                        vr, b + (qq * HD + 32 * w + r32) * 16 + 8 * s, 0, 0));
        }
    };

    const int prow = pos0 + t0 + (r32 >> 3);  // position of the lane's row
    const int plo = window_lo(prow, win);
    float m_run = NEG_INF, l_run = 0.f;
    f32x16 O = f32x16{};
    auto step = [&](TileRegs<FMT>& X, int j) {
        const int k0 = lo + j * TILE;
        f32x16 S = f32x16{};
        if constexpr (FMT == 1) {
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const f32x4 qv = *(const f32x4*)&qs[r32][32 * w + 8 * m + 4 * s];
#pragma unroll
                for (int b = 0; b < 4; b++) S = mfma32f(X.k[m][b], qv[b], S);
            }
        } else {
#pragma unroll
            for (int a = 0; a < 2; a++) {
                const f32x4 q0 = *(const f32x4*)&qs[r32][32 * w + 16 * a + 8 * s];
                const f32x4 q1 = *(const f32x4*)&qs[r32][32 * w + 16 * a + 8 * s + 4];
#pragma unroll
                for (int b = 0; b < 4; b++) S = mfma32f((float)X.k[a][b], q0[b], S);
#pragma unroll
                for (int b = 0; b < 4; b++) S = mfma32f((float)X.k[a][4 + b], q1[b], S);
            }
        }
        const int pb = (j / NWG) & 1;
        f32x4(&sg)[4][4][64] = sx[pb][grp];
#pragma unroll
        for (int a = 0; a < 4; a++) sg[w][a][lane] = f32x4{S[4 * a], S[4 * a + 1], S[4 * a + 2], S[4 * a + 3]};
        lds_barrier();
        float sv[16];
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const f32x4 p0 = sg[0][a][lane], p1 = sg[1][a][lane], p2 = sg[2][a][lane], p3 = sg[3][a][lane];
#pragma unroll
            for (int b = 0; b < 4; b++) sv[4 * a + b] = (p0[b] + p1[b]) + (p2[b] + p3[b]);
        }
        float mt = NEG_INF;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int key = k0 + 8 * (i >> 2) + 4 * s + (i & 3);
            sv[i] = (key >= plo && key <= prow && key < hi) ? sv[i] * scale2 : NEG_INF;
            mt = fmaxf(mt, sv[i]);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(m_run, mt);
        const float base = mn == NEG_INF ? 0.f : mn;
        const float cf = m_run == NEG_INF ? 0.f : exp2f(m_run - mn);
        float ls = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            sv[i] = exp2f(sv[i] - base);
            ls += sv[i];
        }
        ls += __shfl_xor(ls, 32);
        l_run = l_run * cf + ls;
        m_run = mn;
        if (__builtin_amdgcn_ballot_w64(cf != 1.f)) {
#pragma unroll
            for (int i = 0; i < 16; i++) O[i] *= __shfl(cf, 8 * (i >> 2) + 4 * s + (i & 3));
        }
        float vv[4][4];
#pragma unroll
        for (int qq = 0; qq < 4; qq++)
#pragma unroll
            for (int b = 0; b < 4; b++) vv[qq][b] = (float)X.v[qq][b];
        // positions outside [lo_first, hi) may be rows of other positions or never written: P is 0 there, and V
        // must not bring NaN in
        if (k0 < lo_first || k0 + TILE > hi) {
#pragma unroll
            for (int qq = 0; qq < 4; qq++)
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const int key = k0 + 8 * qq + 4 * s + b;
                    if (key < lo_first || key >= hi) vv[qq][b] = 0.f;
                }
        }
#pragma unroll
        for (int qq = 0; qq < 4; qq++)
#pragma unroll
            for (int b = 0; b < 4; b++) O = mfma32f(sv[4 * qq + b], vv[qq][b], O);
    };

    const int rounds = (ntile + NWG - 1) / NWG;
    TileRegs<FMT> A, B;
    load(A, grp);
    for (int i = 0; i < rounds; i += 2) {
        load(B, (i + 1) * NWG + grp);
        step(A, i * NWG + grp);
        if (i + 1 >= rounds) break;
        load(A, (i + 2) * NWG + grp);
        step(B, (i + 1) * NWG + grp);
    }

    if constexpr (NWG == 2) {  // group 1's state into group 0 through LDS
        __syncthreads();
        float* ob = (float*)&sx[0][0][0][0][0];  // [wave][16][64], then m, l of 32 rows
        float* ml = ob + 4 * 16 * 64;
        if (grp == 1) {
#pragma unroll
            for (int i = 0; i < 16; i++) ob[(w * 16 + i) * 64 + lane] = O[i];
            if (w == 0 && s == 0) {
                ml[r32] = m_run;
                ml[32 + r32] = l_run;
            }
        }
        __syncthreads();
        if (grp == 1) return;
        const float m1 = ml[r32], l1 = ml[32 + r32];
        const float M = fmaxf(m_run, m1);
        const float f0 = m_run == NEG_INF ? 0.f : exp2f(m_run - M), f1 = m1 == NEG_INF ? 0.f : exp2f(m1 - M);
        l_run = l_run * f0 + l1 * f1;
        m_run = M;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int row = 8 * (i >> 2) + 4 * s + (i & 3);
            O[i] = O[i] * __shfl(f0, row) + ob[(w * 16 + i) * 64 + lane] * __shfl(f1, row);
        }
    }

    // partials [kvh][row < 8T][split][PART], row = token * 8 + head of the kv head
    const size_t rbase = (size_t)kvh * T * GQA + (size_t)t0 * GQA;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int row = 8 * (i >> 2) + 4 * s + (i & 3);
        if (t0 + (row >> 3) < T) part[((rbase + row) * nch + c) * PART + PACC + 32 * w + r32] = O[i];
    }
    if (w == 0 && s == 0 && t0 + (r32 >> 3) < T) {
        float* p = part + ((rbase + r32) * nch + c) * PART;
        p[0] = m_run;
        p[1] = l_run;
    }
}

// Merge of the splits with the sink (attn_fd_merge, flint_attn.wgsl:241-257): M = max(sink, m_c), out =
// sum_c 2^(m_c - M) acc_c / (2^(sink - M) + sum_c 2^(m_c - M) l_c), all in log2 units. 8 rows (token, head) per
// work-group of 256 threads, 4 dims per thread.
__global__ void __launch_bounds__(256) fl_merge(const float* __restrict__ part, int T, int nch,
                                                const float* __restrict__ sinks, float* __restrict__ out) {
    const int rowid = blockIdx.x * 8 + (threadIdx.x >> 5);  // t * 32 + head
    if (rowid >= T * QH) return;
    const int t = rowid / QH, head = rowid % QH, d0 = (threadIdx.x & 31) * 4;
    const float* p = part + ((size_t)(head / GQA) * T * GQA + (size_t)t * GQA + head % GQA) * nch * PART;
    float M = sinks ? sinks[head] * LOG2E : NEG_INF;
    for (int c = 0; c < nch; c++) M = fmaxf(M, p[(size_t)c * PART]);
    float Lsum = sinks && M != NEG_INF ? exp2f(sinks[head] * LOG2E - M) : 0.f;
    f32x4 acc = f32x4{};
#pragma unroll 4
    for (int c = 0; c < nch; c++) {
        const float* pc = p + (size_t)c * PART;
        const float mc = pc[0];
        const float e = mc == NEG_INF ? 0.f : exp2f(mc - M);
        Lsum += e * pc[1];
        const f32x4 a = *(const f32x4*)(pc + PACC + d0);
        acc += e * a;
    }
    *(f32x4*)(out + ((size_t)t * QH + head) * HD + d0) = acc / Lsum;
}

// K and V rows of ntok tokens into ring rows (pos0 + t) % rows: items (token, kv head, 8 dims).
template <int FMT>
__global__ void __launch_bounds__(256) fl_append(void* __restrict__ kplane, void* __restrict__ vplane,
                                                 size_t plane_elems, int rows, int pos0, int ntok,
                                                 const float* __restrict__ k, const float* __restrict__ v) {
    const int id = blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= ntok * KVH * (HD / 8)) return;
    const int t = id / (KVH * HD / 8), kh = (id / (HD / 8)) % KVH, d0 = (id % (HD / 8)) * 8;
    const int r = (pos0 + t) % rows;
    const float* ks = k + ((size_t)t * KVH + kh) * HD + d0;
    const float* vs = v + ((size_t)t * KVH + kh) * HD + d0;
    if constexpr (FMT == 1) {
        float* kp = (float*)kplane + (size_t)kh * plane_elems;
        float* vp = (float*)vplane + (size_t)kh * plane_elems;
        *(f32x4*)(kp + k_off(r, d0)) = *(const f32x4*)ks;
        *(f32x4*)(kp + k_off(r, d0 + 4)) = *(const f32x4*)(ks + 4);
#pragma unroll
        for (int j = 0; j < 8; j++) vp[v_off32(r, d0 + j)] = vs[j];
    } else {
        unsigned short* kp = (unsigned short*)kplane + (size_t)kh * plane_elems;
        unsigned short* vp = (unsigned short*)vplane + (size_t)kh * plane_elems;
        u16x8 kw;
#pragma unroll
        for (int j = 0; j < 8; j++) kw[j] = f2h(ks[j]);
        *(u16x8*)(kp + k_off16(r, d0)) = kw;
#pragma unroll
        for (int j = 0; j < 8; j++) vp[v_off16(r, d0 + j)] = f2h(vs[j]);
    }
}

// NEOX RoPE: work-group (token, head), thread i rotates the pair (i, i + 64) (rope_neox_n, flint_attn.wgsl:49-57).
__global__ void __launch_bounds__(64) fl_rope(int heads, const float* __restrict__ x, const float* __restrict__ tab,
                                              float* __restrict__ out) {
#pragma clang fp contract(off)
    const int t = blockIdx.x / heads, i = threadIdx.x;
    const size_t h0 = (size_t)blockIdx.x * HD;
    const float x0 = x[h0 + i], x1 = x[h0 + i + 64];
    const float cs = tab[(size_t)t * HD + i], sn = tab[(size_t)t * HD + 64 + i];
    out[h0 + i] = x0 * cs - x1 * sn;
    out[h0 + i + 64] = x0 * sn + x1 * cs;
}

// Store layout <-> the reference's rows [row][kvh][128] for rows [r0, r1) of one layer's K or V.
template <typename E, int DIR>  // DIR 0: store -> rows, 1: rows -> store
__global__ void __launch_bounds__(256) fl_rows(E* __restrict__ plane, size_t plane_elems, E* __restrict__ rowsbuf,
                                               int r0, int r1, int which) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (size_t)(r1 - r0) * KVH * HD) return;
    const int d = id % HD, kh = (id / HD) % KVH, r = r0 + (int)(id / (KVH * HD));
    constexpr bool F32 = sizeof(E) == 4;
    const size_t o = (size_t)kh * plane_elems +
                     (F32 ? (which == 0 ? k_off(r, d) : v_off32(r, d)) : (which == 0 ? k_off16(r, d) : v_off16(r, d)));
    if (DIR == 0) rowsbuf[id] = plane[o];
    else plane[o] = rowsbuf[id];
}

}  // namespace

Plan plan(int pos0, int T, int win) {
    const int lo0 = win > 0 && pos0 + 1 > win ? pos0 + 1 - win : 0;
    const int klo = lo0 / 32 * 32, span = pos0 + T - klo;
    const int nrb = (T + 3) / 4;
    int nch;
    if (T <= 4) {
        nch = span / 128;  // splits of at least 128 positions, 256 work-groups over the 4 kv heads at most
        nch = nch > 64 ? 64 : nch;
    } else {
        nch = 512 / (nrb * KVH);
        const int most = span / 128;
        nch = nch > most ? most : nch > 16 ? 16 : nch;
    }
    nch = nch < 1 ? 1 : nch;
    return Plan{klo, span, nch, nrb};
}

size_t ws_floats() { return (size_t)KVH * 4096 * PART; }

hipError_t launch_attn(int fmt, const void* kp, const void* vp, int rows, const float* q, int T, int pos0, int win,
                       const Plan& p, float* ws, const float* sinks, float* out, hipStream_t st) {
    if ((size_t)T * GQA * p.nch > 4096) return hipErrorInvalidValue;  // the workspace's rows x splits per kv head
    const size_t pe = (size_t)rows * HD;
    const float scale2 = (1.0f / 11.313708498984761f) * LOG2E;  // 1/sqrt(128) (flint_attn.wgsl:86) in log2 units
    const dim3 grid(p.nrb * p.nch * KVH);
    const Launch L{st};
    hipError_t e;
    if (fmt == 1)
        e = T <= 4 ? launch(fl_attn<1, 1>, grid, dim3(256), L, kp, vp, pe, rows, q, T, pos0, win, scale2, p.klo, p.span,
                            p.nch, p.nrb, ws)
                   : launch(fl_attn<1, 2>, grid, dim3(512), L, kp, vp, pe, rows, q, T, pos0, win, scale2, p.klo, p.span,
                            p.nch, p.nrb, ws);
    else
        e = T <= 4 ? launch(fl_attn<0, 1>, grid, dim3(256), L, kp, vp, pe, rows, q, T, pos0, win, scale2, p.klo, p.span,
                            p.nch, p.nrb, ws)
                   : launch(fl_attn<0, 2>, grid, dim3(512), L, kp, vp, pe, rows, q, T, pos0, win, scale2, p.klo, p.span,
                            p.nch, p.nrb, ws);
    if (e != hipSuccess) return e;
    return launch(fl_merge, dim3((T * QH + 7) / 8), dim3(256), L, (const float*)ws, T, p.nch, sinks, out);
}

hipError_t launch_append(int fmt, void* kp, void* vp, int rows, int pos0, int ntok, const float* k, const float* v,
                         hipStream_t st) {
    const int items = ntok * KVH * (HD / 8);
    const dim3 grid((items + 255) / 256);
    const size_t pe = (size_t)rows * HD;
    if (fmt == 1) return launch(fl_append<1>, grid, dim3(256), Launch{st}, kp, vp, pe, rows, pos0, ntok, k, v);
    return launch(fl_append<0>, grid, dim3(256), Launch{st}, kp, vp, pe, rows, pos0, ntok, k, v);
}

hipError_t launch_rope(int ntok, int heads, const float* x, const float* tab, float* out, hipStream_t st) {
    return launch(fl_rope, dim3(ntok * heads), dim3(64), Launch{st}, heads, x, tab, out);
}

hipError_t launch_rows(int fmt, void* plane, int rows, int which, int r0, int r1, void* buf, int dir,
                       hipStream_t st) {
    const size_t total = (size_t)(r1 - r0) * KVH * HD;
    if (total == 0) return hipSuccess;
    const dim3 grid((unsigned)((total + 255) / 256));
    const size_t pe = (size_t)rows * HD;
    const Launch L{st};
    if (fmt == 1)
        return dir == 0 ? launch(fl_rows<float, 0>, grid, dim3(256), L, (float*)plane, pe, (float*)buf, r0, r1, which)
                        : launch(fl_rows<float, 1>, grid, dim3(256), L, (float*)plane, pe, (float*)buf, r0, r1, which);
    return dir == 0 ? launch(fl_rows<unsigned short, 0>, grid, dim3(256), L, (unsigned short*)plane, pe,
                             (unsigned short*)buf, r0, r1, which)
                    : launch(fl_rows<unsigned short, 1>, grid, dim3(256), L, (unsigned short*)plane, pe,
                             (unsigned short*)buf, r0, r1, which);
}

}  // namespace flint
}  // namespace mkv
