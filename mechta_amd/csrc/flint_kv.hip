// flint_kv.hip -- the Flint model's KV path: ring append, NEOX RoPE, conversion to the reference's row layout, and
// sliding-window attention with per-head sinks (flint_attn.wgsl:1-257), for one decode token or a prefill block.
//
// Three attention kernels: fl_dec16 (1-2 tokens, 16 query rows), fl_attn (3-4 tokens) and fl_pf (prefill blocks of
// 5-512 tokens, 32 tokens per work-group sharing an LDS ring of K/V tiles). fl_attn's work-group: (block of 4 tokens,
// key split, kv head) = 32 query rows (token * 8 + head) against the split's keys in tiles of 32 positions. The
// arithmetic is f32, as the reference's, taken on the f16 matrix units: f32 operands are split into f16 hi + lo and
// each product is three v_mfma_f32_32x32x16_f16 passes (hi.hi + hi.lo + lo.hi, f32 accumulation), two where one side
// is an f16 cache's K or V (exact in f16). Per tile, wave w of 4:
//   S^T[32 keys][32 rows] over dims 32w .. 32w+31    2 dim steps, A = K straight from HBM, B = Q (split once, LDS)
//   the four partial S^T summed through LDS in one order, exact-max online softmax (redundantly in every wave)
//   O[32 rows][dims 32w .. 32w+31] += P . V           2 key steps, A = P (split from the S^T registers), B = V
// The 32x32 accumulator layout gives lane l (half s = l / 32) row l % 32 and keys 8a + 4s + b (register 4a + b), the
// keys a 16-key step k of P.V takes in lane half s (16k + 4s + b and 16k + 8 + 4s + b: the order within a step is
// free as long as P and V agree); with V stored in groups of 4 (f32) or 8 (f16) positions each register quad's keys
// are one 16-byte (f32) or 8-byte (f16) load. Rows are positions modulo the ring: a 32-position
// tile is one 32-row block (rings are multiples of 32), so a ring wrap only changes the tile's base address.
// Each split writes one partial [m, l, 0, 0, acc[128]] per row; fl_merge adds the sink (as attn_fd_merge,
// flint_attn.wgsl:241-257: the sink joins the maximum and the sum, never the output) and normalizes.
#include "flint_internal.h"
#include "mkv_device.h"

namespace mkv {
namespace flint {
namespace {

#ifndef FL_DEC_BUF
#define FL_DEC_BUF 2      // decode: subtiles in registers per wave
#endif
#ifndef FL_DEC_SPLIT
#define FL_DEC_SPLIT 32   // decode: positions per split at least
#endif
#ifndef FL_DEC_NCH
#define FL_DEC_NCH 48     // decode: splits per kv head at most (32,768 positions: 48 against 32 / 64 / 96 splits
                          // 17.9-18.3 against 19.2 / 18.3-18.5 / 19.7 us per f16 call)
#endif
#ifndef FL_FUSE_NCH
#define FL_FUSE_NCH 8     // decode with the merge fused (short spans): splits per kv head at most
#endif
#ifndef FL_FUSE_SPLIT
#define FL_FUSE_SPLIT 80  // decode with the merge fused: positions per split at least (at 544 positions: 6 splits;
                          // against 8 / 7 / 5 / 4 splits 9.8 against 10.7 / 9.8 / 10.0 / 10.7 us per f32 call, 8.6
                          // against 8.8 / 8.6 / 8.5 / 8.8 us per f16 call)
#endif
// Decodes of spans up to these many positions merge in the kernel; longer ones launch the merge. One token on a full
// layer, us per call with the merge in the kernel against two launches: f32 at 320 / 384 / 448 / 512 / 768 / 2,048
// positions 9.1 / 9.5 / 10.1 / 10.2 / 10.4 / 13.0 against 9.0 / 9.5 / 9.8 / 9.9 / 9.6 / 10.7; f16 8.1 / 8.3 / 8.6 / 8.8
// / 9.0 / 10.4 against 8.2 / 8.6 / 8.8 / 9.0 / 8.7 / 9.2; at 256 positions 9.0 / 8.2 against 10.7 / 10.2 (f32 / f16).
// A sliding layer's 513-544 positions: 9.8 / 8.6 against 8.9 / 8.3.
#ifndef FL_FUSE_SPAN_F32
#define FL_FUSE_SPAN_F32 384
#endif
#ifndef FL_FUSE_SPAN_F16
#define FL_FUSE_SPAN_F16 512
#endif

constexpr int TILE = 32;
constexpr int QPAD = HD + 8;  // LDS row of Q's halves: 16-byte reads of 32 rows conflict-free


// Window start of the token at position p: the 513 positions up to p on sliding layers (lo_di, flint_attn.wgsl:82).
__device__ inline int window_lo(int p, int win) { return win > 0 && p + 1 > win ? p + 1 - win : 0; }

template <int FMT>
struct TileRegs;
template <>
struct TileRegs<1> {  // f32: K dims 32w + 16a + 8s + 4e .. +3 of key l % 32 (index 2a + e); V keys 8q + 4s .. +3 of
                      // dim 32w + l % 32
    f32x4 k[4];
    f32x4 v[4];
};
template <>
struct TileRegs<0> {  // f16: K dims 32w + 16a + 8s .. +7 (a < 2); V keys 8q + 4s .. +3, 4 halves
    half8 k[2];
    half4 v[4];
};

template <int FMT, int NBUF>  // NBUF: tiles in registers (NBUF - 1 in flight ahead of the one computed)
__global__ void __launch_bounds__(256) fl_attn(const void* __restrict__ kplane, const void* __restrict__ vplane,
                                               size_t plane_elems, int rows, const float* __restrict__ q, int T,
                                               int pos0, int win, float scale2, int klo, int span, int nch, int nrb,
                                               float* __restrict__ part) {
    constexpr int BPE = FMT == 1 ? 4 : 2;
    constexpr unsigned TILE_BYTES = TILE * HD * BPE;
    const int G = gridDim.x, L = blockIdx.x;
    const int W = G % NXCD == 0 ? (L % NXCD) * (G / NXCD) + L / NXCD : L;
    const int rb = W % nrb, c = (W / nrb) % nch, kvh = W / nrb / nch;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, s = lane >> 5, r32 = lane & 31;
    const int t0 = 4 * rb, nt = min(4, T - t0);
    const int lo_first = window_lo(pos0 + t0, win);  // the block's earliest visible position
    const int cs = klo + chunk_lo(c, span, nch), ce = c + 1 < nch ? klo + chunk_lo(c + 1, span, nch) : klo + span;
    const int lo = max(cs, lo_first / TILE * TILE), hi = min(ce, pos0 + t0 + nt);  // keys [lo, hi) of this split
    const int ntile = hi > lo ? (hi - lo + TILE - 1) / TILE : 0;

    __shared__ __attribute__((aligned(16))) _Float16 qh[32][QPAD], ql[32][QPAD];  // Q split: hi, lo
    __shared__ f32x4 sx[2][4][4][64];  // partial S^T: [tile parity][wave][register quad][lane]
    for (int i = tid; i < 32 * HD / 8; i += 256) {
        const int row = i / (HD / 8), d8 = (i % (HD / 8)) * 8, t = t0 + (row >> 3);
        f32x4 x0 = f32x4{}, x1 = f32x4{};
        if (t < T) {
            const float* qr = q + ((size_t)t * QH + kvh * GQA + (row & 7)) * HD + d8;
            x0 = *(const f32x4*)qr;
            x1 = *(const f32x4*)(qr + 4);
        }
        half8 hi, lo;
        split8(x0, x1, hi, lo);
        *(half8*)&qh[row][d8] = hi;
        *(half8*)&ql[row][d8] = lo;
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
                    kr, b + ((8 * w + 4 * (m >> 1) + 2 * s + (m & 1)) * TILE + r32) * 16, 0, LOAD_NT));
#pragma unroll
            for (int qq = 0; qq < 4; qq++)
                X.v[qq] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        vr, b + ((2 * qq + s) * HD + 32 * w + r32) * 16, 0, LOAD_NT));
        } else {
#pragma unroll
            for (int a = 0; a < 2; a++)
                X.k[a] = bload16(kr, b + ((4 * w + 2 * a + s) * TILE + r32) * 16);
#pragma unroll
            for (int qq = 0; qq < 4; qq++)
                X.v[qq] = __builtin_bit_cast(half4, __builtin_amdgcn_raw_buffer_load_b64(
                                                        vr, b + (qq * HD + 32 * w + r32) * 16 + 8 * s, 0, LOAD_NT));
        }
    };

    const int prow = pos0 + t0 + (r32 >> 3);  // position of the lane's row
    const int plo = window_lo(prow, win);
    float m_run = NEG_INF, l_run = 0.f;
    f32x16 O = f32x16{};
    auto step = [&](TileRegs<FMT>& X, int j) {
        const int k0 = lo + j * TILE;
        f32x16 S = f32x16{};
#pragma unroll
        for (int a = 0; a < 2; a++) {  // dims 32w + 16a .. +15, lane half s: 8s .. 8s + 7
            const half8 bh = *(const half8*)&qh[r32][32 * w + 16 * a + 8 * s];
            const half8 bl = *(const half8*)&ql[r32][32 * w + 16 * a + 8 * s];
            if constexpr (FMT == 1) {
                half8 kh, kl;
                split8(X.k[2 * a], X.k[2 * a + 1], kh, kl);
                S = mfma3(kh, kl, bh, bl, S);
            } else {
                S = mfma2(X.k[a], bh, bl, S);
            }
        }
        f32x4(&sg)[4][4][64] = sx[j & 1];
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
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int key = k0 + 8 * (i >> 2) + 4 * s + (i & 3);
            sv[i] = (key >= plo && key <= prow && key < hi) ? sv[i] * scale2 : NEG_INF;
        }
        float mt = vmax(sv[0], sv[1]);  // masked scores are -inf, never NaN: single-instruction maxima
#pragma unroll
        for (int i = 2; i < 16; i += 2) mt = vmax3(mt, sv[i], sv[i + 1]);
        mt = max_xor32(mt);
        const float mn = fmaxf(m_run, mt);
        const float base = mn == NEG_INF ? 0.f : mn;
        const float cf = m_run == NEG_INF ? 0.f : fast_exp2(m_run - mn);
        float ls = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            sv[i] = fast_exp2(sv[i] - base);
            ls += sv[i];
        }
        ls = add_xor32(ls);
        l_run = l_run * cf + ls;
        m_run = mn;
        if (__builtin_amdgcn_ballot_w64(cf != 1.f)) {
#pragma unroll
            for (int i = 0; i < 16; i++) O[i] *= __shfl(cf, 8 * (i >> 2) + 4 * s + (i & 3));
        }
        // positions outside [lo_first, hi) may be rows of other positions or never written: P is 0 there, and V
        // must not bring NaN in
        if (k0 < lo_first || k0 + TILE > hi) {
#pragma unroll
            for (int qq = 0; qq < 4; qq++)
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const int key = k0 + 8 * qq + 4 * s + b;
                    if (key < lo_first || key >= hi) {
                        if constexpr (FMT == 1) X.v[qq][b] = 0.f;
                        else X.v[qq][b] = (_Float16)0.f;
                    }
                }
        }
#pragma unroll
        for (int k = 0; k < 2; k++) {  // keys 16k + 4s + b (registers 8k + b) and 16k + 8 + 4s + b (8k + 4 + b)
            half8 ph, pl;
            split8(f32x4{sv[8 * k], sv[8 * k + 1], sv[8 * k + 2], sv[8 * k + 3]},
                   f32x4{sv[8 * k + 4], sv[8 * k + 5], sv[8 * k + 6], sv[8 * k + 7]}, ph, pl);
            if constexpr (FMT == 1) {
                half8 vh, vl;
                split8(X.v[2 * k], X.v[2 * k + 1], vh, vl);
                O = mfma3(ph, pl, vh, vl, O);
            } else {
                const half8 vb = __builtin_shufflevector(X.v[2 * k], X.v[2 * k + 1], 0, 1, 2, 3, 4, 5, 6, 7);
                O = mfma32(pl, vb, mfma32(ph, vb, O));
            }
        }
    };

    // a ring of NBUF register tiles: round r computes slot r % NBUF after issuing the loads of round r + NBUF - 1
    // into the slot round r - 1 freed (the slots are unrolled, so every index is a constant)
    const int rounds = ntile;
    TileRegs<FMT> R[NBUF];
#pragma unroll
    for (int k = 0; k < NBUF - 1; k++) load(R[k], k);
    for (int i0 = 0; i0 < rounds; i0 += NBUF) {
#pragma unroll
        for (int k = 0; k < NBUF; k++) {
            if (i0 + k < rounds) {  // uniform in the work-group
                load(R[(k + NBUF - 1) % NBUF], i0 + k + NBUF - 1);
                step(R[k], i0 + k);
            }
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

// Prefill: work-group = (32 tokens of the block, key split, kv head), 8 waves of 4 tokens x 8 heads = 32 query rows
// each. The split's 32-key tiles (K and V of 32 positions, each contiguous: a tile is one 32-row block of the ring)
// stream through an LDS ring filled by direct global->LDS loads and shared by the 8 waves, so a key is fetched once
// per 32 tokens, not once per 4. Per tile and wave:
//   S^T[32 keys][32 rows] = K . Q^T   8 dim steps of v_mfma_f32_32x32x16_f16 (A = K rows in key_perm order from
//                                     LDS; B = Q split hi + lo, in registers for the whole split): 2 passes on an
//                                     f16 cache (K exact), 3 on an f32 cache (each ring slot's K and V split into
//                                     f16 hi + lo once, in place, by the whole work-group)
//   online softmax in registers with a lazy reference max (moves when first or when the tile maximum exceeds it by
//   more than 8; the partial's m is that reference, which the merge treats like any other), f32 P
//   O[32 rows][128] += P . V          2 key steps x 4 dim blocks (A = P split hi + lo from the S registers, B = V
//                                     from LDS): 2 passes (f16 V exact) or 3 (f32 V split)
// The result is the same f32-class arithmetic as fl_attn; only the summation order differs.
#ifndef FL_PF_SUB16
#define FL_PF_SUB16 2
#endif
#ifndef FL_PF_SUB32
#define FL_PF_SUB32 1
#endif
#ifndef FL_PF_NSLOT
#define FL_PF_NSLOT 4
#endif
constexpr int PF_NW = 8;               // waves per work-group
constexpr int PF_PT = 4 * PF_NW;       // tokens per work-group
constexpr int PF_NSLOT = FL_PF_NSLOT;  // ring slots: PF_NSLOT - 1 in flight

template <int FMT>
struct PfGeom {
    static constexpr int BPE = FMT == 1 ? 4 : 2;
    static constexpr int SUB = FMT == 1 ? FL_PF_SUB32 : FL_PF_SUB16;  // 32-key tiles per ring slot (per barrier)
    static constexpr int TILE_BYTES = TILE * HD * BPE;                // K (or V) bytes of one tile
    static constexpr int SLOT = 2 * SUB * TILE_BYTES;                 // K tiles, then V tiles of a slot
    static constexpr int DPT = TILE_BYTES / PF_NW / 1024;             // direct loads per wave and K (or V) tile
    static constexpr int LPT = 2 * SUB * DPT;                         // direct loads per wave and slot
    static constexpr int EPG = 16 / BPE;                              // positions per V group
    static_assert((PF_NSLOT - 2) * LPT <= 63, "vmcnt range");
};

template <int N>
__device__ inline void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
template <int L, int LPT>  // wait until at most `later` slots (LPT direct loads each) of this wave are pending
__device__ inline void pf_wait(int later) {
    if constexpr (L == 0) {
        vm_wait<0>();
    } else {
        if (later >= L) vm_wait<L * LPT>();
        else pf_wait<L - 1, LPT>(later);
    }
}

template <int FMT>
__global__ void __launch_bounds__(PF_NW * 64) fl_pf(const void* __restrict__ kplane, const void* __restrict__ vplane,
                                                    size_t plane_elems, int rows, const float* __restrict__ q, int T,
                                                    int pos0, int win, float scale2, int klo, int span, int nch,
                                                    float* __restrict__ part) {
    using Gm = PfGeom<FMT>;
    constexpr int SUB = Gm::SUB, TB = Gm::TILE_BYTES, SLOT = Gm::SLOT;
    // XCD-aware order (as the decode and prefill kernels): the token blocks of one (split, kv head) on one XCD
    const int G = gridDim.x, Lb = blockIdx.x;
    const int W = G % NXCD == 0 ? (Lb % NXCD) * (G / NXCD) + Lb / NXCD : Lb;
    const int nblk = (T + PF_PT - 1) / PF_PT;
    const int rb = W % nblk, c = (W / nblk) % nch, kvh = W / nblk / nch;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, r = lane & 31;
    const int tb = rb * PF_PT, tlast = min(T - 1, tb + PF_PT - 1);
    const int lo_first = window_lo(pos0 + tb, win);  // the block's earliest visible position
    const int kend = pos0 + tlast + 1;               // keys [lo_first, kend) hold the block's positions
    // the split divides this block's own keys [blo, bhi), not the call's: on a sliding layer each block's window is
    // 544 of the call's 1,024 positions, and splits of the call's range gave one work-group 8 tiles and another none
    // (512 tokens: 36.8 -> 32.1 us per f32 call, 30.3 -> 28.0 us f16)
    const int blo = max(klo, lo_first / TILE * TILE), bhi = min(klo + span, kend);  // tile-aligned start
    const int bsp = bhi > blo ? bhi - blo : 0;
    const int lo = blo + chunk_lo(c, bsp, nch), hi = c + 1 < nch ? blo + chunk_lo(c + 1, bsp, nch) : bhi;
    const int nt32 = hi > lo ? (hi - lo + TILE - 1) / TILE : 0;
    const int ntiles = (nt32 + SUB - 1) / SUB;  // ring slots to stream
    const unsigned char* K = (const unsigned char*)kplane + (size_t)kvh * plane_elems * Gm::BPE;
    const unsigned char* V = (const unsigned char*)vplane + (size_t)kvh * plane_elems * Gm::BPE;

    __shared__ __attribute__((aligned(16))) unsigned char ring[PF_NSLOT * SLOT];
    __shared__ __attribute__((aligned(16))) float cfs[PF_NW][32];  // rescale factors of a wave's rows
    // Each wave copies 1/8 of every K and V tile of slot j: K bytes [w TB/8, +TB/8). V: f16, the same; f32, dims
    // [64 (w % 2), +64) of groups 2 (w / 2) and 2 (w / 2) + 1 (1 KB each), so that the V chunk pairs the wave splits
    // below are its own copies (K's are in either layout).
    const unsigned kreg = w * (TB / PF_NW);
    const unsigned vreg0 = FMT == 1 ? (2 * (w >> 1)) * (HD * 16) + (w & 1) * (HD / 2 * 16) : kreg;
    // per-lane offsets of the wave's regions, fixed for the kernel; the tile's base and LDS slot are wave-uniform
    const unsigned vk = kreg + lane * 16, vv = vreg0 + lane * 16;
    const unsigned lk = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_void*)ring + kreg);
    const unsigned lv = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_void*)ring + vreg0);
    auto issue = [&](int j) {
        const unsigned slot = (j % PF_NSLOT) * SLOT;
#pragma unroll
        for (int u = 0; u < SUB; u++) {
            // a 32-position tile is one 32-row block of the ring (rows are a multiple of 32), K and V alike; tiles
            // past the split's end stay inside the plane and are never computed
            const size_t off = (size_t)((lo + TILE * (SUB * j + u)) % rows) * HD * Gm::BPE;
#pragma unroll
            for (int d = 0; d < Gm::DPT; d++) {
                dma16s(K + off + d * 1024, vk, lk + slot + u * TB + d * 1024);
                // f32: d = 0, 1 are the two groups' 1 KB (DPT = 2); f16: the wave's 1 KB parts in order
                const unsigned vd = FMT == 1 ? d * (HD * 16) : d * 1024;
                dma16s(V + off + vd, vv, lv + slot + (SUB + u) * TB + vd);
            }
        }
    };
    for (int j = 0; j < PF_NSLOT - 1 && j < ntiles; j++) issue(j);

    // Q as the B operand of S^T: lane (r, h) holds row r (token tr, head r % 8), dims 16s + 8h .. +7 of step s, split
    // into f16 hi + lo; rows of tokens past the block are zero and see no key
    const int tr = tb + 4 * w + (r >> 3);
    const int vlo = tr < T ? window_lo(pos0 + tr, win) : 0, vhi = tr < T ? pos0 + tr + 1 : 0;  // row sees [vlo, vhi)
    half8 qh[8], ql[8];
    {
        const float* qrow = q + ((size_t)min(tr, T - 1) * QH + kvh * GQA + (r & 7)) * HD + 8 * h;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            f32x4 x0 = *(const f32x4*)(qrow + 16 * s), x1 = *(const f32x4*)(qrow + 16 * s + 4);
            if (tr >= T) x0 = x1 = f32x4{};
            split8(x0, x1, qh[s], ql[s]);
        }
    }
    // K in a tile: f16 [dims/8][32 keys][8], f32 [dims/4][32 keys][4]; lane (r, h) of step s takes dims 16s + 8h .. +7
    // of key key_perm(r)
    const int kaddr = FMT == 1 ? h * 1024 + key_perm(r) * 16 : h * 512 + key_perm(r) * 16;
    float m = NEG_INF, lsum = 0.f;
    f32x16 O[4];
#pragma unroll
    for (int nb = 0; nb < 4; nb++) O[nb] = f32x16{};

    // V rows of a slot outside [lo_first, kend) may be other positions' or never written: zero them in LDS so that
    // 0 * V stays finite (K there only meets masked scores)
    auto zero_v = [&](int j) {
        constexpr int EPG = Gm::EPG;
        unsigned char* Vz = ring + (j % PF_NSLOT) * SLOT + SUB * TB;
        const int k0 = lo + TILE * SUB * j;
        for (int i = tid; i < SUB * TILE * HD; i += PF_NW * 64) {
            const int key = k0 + (i / (EPG * HD)) * EPG + (i % EPG);  // V group i / (EPG * HD), position i % EPG
            if (key < lo_first || key >= kend) {
                if constexpr (FMT == 1) ((float*)Vz)[i] = 0.f;
                else ((unsigned short*)Vz)[i] = 0;
            }
        }
    };
    for (int j = 0; j < ntiles; j++) {
        pf_wait<PF_NSLOT - 2, Gm::LPT>(min(ntiles - 1 - j, PF_NSLOT - 2));  // this wave's copies of slot j landed
        const int ks0 = lo + TILE * SUB * j;
        if constexpr (FMT == 1) {
            // this wave's part of the slot's f32 K and V split once, in place, into f16 hi + lo (the 8 waves then read
            // split operands instead of each splitting the same tiles): a pair of 16-byte chunks holds 8 consecutive
            // dims of one key (K chunks d/4 = 2g, 2g + 1) or 8 consecutive keys of one dim (V groups 2g, 2g + 1); hi
            // goes over the first chunk and lo over the second, where the operand reads find them. The pairs are the
            // ones this wave copied, so no barrier comes between its copies and its split. V rows outside
            // [lo_first, kend) are zeroed on the way (0 * V stays finite).
            static_assert(TB / PF_NW == 2048 && HD / 2 * 16 == 1024, "2 KB of K and 2 x 1 KB of V per wave");
            unsigned char* sl = ring + (j % PF_NSLOT) * SLOT;
#pragma unroll
            for (int u = 0; u < SUB; u++) {
                // K pair: chunk 4w + 2 (lane / 32) of key lane % 32; V pair: dim 64 (w % 2) + lane of groups 2 (w / 2), +1
                unsigned char* a = sl + u * TB + ((4 * w + 2 * (lane >> 5)) * 32 + (lane & 31)) * 16;
                half8 kh, kl;
                split8(*(const f32x4*)a, *(const f32x4*)(a + 512), kh, kl);
                unsigned char* b = sl + (SUB + u) * TB + vreg0 + lane * 16;
                f32x4 v0 = *(const f32x4*)b, v1 = *(const f32x4*)(b + HD * 16);
                const int key = ks0 + TILE * u + 8 * (w >> 1);
                if (key < lo_first || key + 8 > kend) {
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        v0[e] = key + e >= lo_first && key + e < kend ? v0[e] : 0.f;
                        v1[e] = key + 4 + e >= lo_first && key + 4 + e < kend ? v1[e] : 0.f;
                    }
                }
                half8 vh, vl;
                split8(v0, v1, vh, vl);
                *(half8*)a = kh;
                *(half8*)(a + 512) = kl;
                *(half8*)b = vh;
                *(half8*)(b + HD * 16) = vl;
            }
        }
        lds_barrier();  // slot j is in LDS (f32: split) for every wave; every wave is done with slot j - 1
        if (j + PF_NSLOT - 1 < ntiles) issue(j + PF_NSLOT - 1);  // into the slot of j - 1
        if (FMT == 0 && (ks0 < lo_first || ks0 + TILE * SUB > kend)) {
            zero_v(j);
            lds_barrier();
        }
#pragma unroll
        for (int u = 0; u < SUB; u++) {
            const int k0 = ks0 + TILE * u;
            if (k0 >= hi) break;
            const unsigned char* Ks = ring + (j % PF_NSLOT) * SLOT + u * TB;
            const unsigned char* Vs = ring + (j % PF_NSLOT) * SLOT + (SUB + u) * TB;
            // independent chains (Q hi; Q lo and K lo), added once: back-to-back MFMAs never wait on each other
            f32x16 Sh = f32x16{}, Sl = f32x16{};
            if constexpr (FMT == 1) {
                constexpr int KP = 2;  // K operands (hi and lo, split in the ring) in flight ahead of the MFMAs
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
            } else {
                constexpr int KP = 3;  // K operands in flight ahead of the MFMAs
                half8 kbuf[KP];
#pragma unroll
                for (int s = 0; s < KP; s++) kbuf[s] = *(const half8*)(Ks + kaddr + s * 1024);
#pragma unroll
                for (int s = 0; s < 8; s++) {
                    const half8 ka = kbuf[s % KP];
                    if (s + KP < 8) kbuf[s % KP] = *(const half8*)(Ks + kaddr + (s + KP) * 1024);
                    Sh = mfma32(ka, qh[s], Sh);
                    Sl = mfma32(ka, ql[s], Sl);
                }
                __builtin_amdgcn_sched_group_barrier(0x100, KP, 0);
#pragma unroll
                for (int s = 0; s < 8 - KP; s++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 2 * KP, 0);
            }
            f32x16 S = Sh + Sl;
            // register i of lane (r, h) is key 8h + i (i < 8) or 16 + 8h + i - 8 of the tile for row r
            if (!__all(k0 >= vlo && k0 + TILE <= vhi)) {
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int key = k0 + 8 * h + i + (i >= 8 ? 8 : 0);
                    S[i] = (key >= vlo && key < vhi) ? S[i] : NEG_INF;
                }
            }
            // masked scores are -inf, never NaN: single-instruction maxima after the first, which is the compiler's
            // (it reads the MFMA results and so carries the wait states a vector read of them needs)
            float mt = fmaxf(S[0], S[1]);
#pragma unroll
            for (int i = 2; i < 16; i += 2) mt = vmax3(mt, S[i], S[i + 1]);
            mt = max_xor32(mt);
            mt *= scale2;  // scale2 > 0: the max of the scaled scores is the scaled max
            const bool rescale = m != NEG_INF && mt > m + LAZY2;
            const float mr = m == NEG_INF || rescale ? fmaxf(m, mt) : m;
            float cf = 1.f;
            if (__any(rescale)) {
                // register i of O holds row 8(i/4) + 4h + i%4, whose factor lane (that row) holds: the 32 factors
                // pass through this wave's LDS row
                cf = rescale ? fast_exp2(m - mr) : 1.f;
                if (h == 0) cfs[w][r] = cf;
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int a = 0; a < 4; a++) {
                    const f32x4 f = *(const f32x4*)&cfs[w][8 * a + 4 * h];
#pragma unroll
                    for (int nb = 0; nb < 4; nb++) {
#pragma unroll
                        for (int qq = 0; qq < 4; qq++) O[nb][4 * a + qq] *= f[qq];
                    }
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
            // key step k: keys 16k + 8h .. +7 (f16: V group 2k + h; f32: groups 4k + 2h, +1); dim block nb: 32nb + r
            if constexpr (FMT == 1) {
                auto vaddr = [&](int i) { return Vs + (4 * (i >> 2) + 2 * h) * (HD * 16) + (32 * (i & 3) + r) * 16; };
                constexpr int VP = 2;
                half8 vbuf[VP][2];
#pragma unroll
                for (int i = 0; i < VP; i++) {
                    vbuf[i][0] = *(const half8*)vaddr(i);
                    vbuf[i][1] = *(const half8*)(vaddr(i) + HD * 16);
                }
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const half8 vh = vbuf[i % VP][0], vl = vbuf[i % VP][1];
                    if (i + VP < 8) {
                        vbuf[i % VP][0] = *(const half8*)vaddr(i + VP);
                        vbuf[i % VP][1] = *(const half8*)(vaddr(i + VP) + HD * 16);
                    }
                    O[i & 3] = mfma32(pl[i >> 2], vh, mfma32(ph[i >> 2], vl, mfma32(ph[i >> 2], vh, O[i & 3])));
                }
            } else {
                half8 vb[8];
#pragma unroll
                for (int i = 0; i < 8; i++)
                    vb[i] = *(const half8*)(Vs + (2 * (i >> 2) + h) * (HD * 16) + (32 * (i & 3) + r) * 16);
#pragma unroll
                for (int k = 0; k < 2; k++) {
#pragma unroll
                    for (int nb = 0; nb < 4; nb++) O[nb] = mfma32(ph[k], vb[4 * k + nb], O[nb]);
#pragma unroll
                    for (int nb = 0; nb < 4; nb++) O[nb] = mfma32(pl[k], vb[4 * k + nb], O[nb]);
                }
            }
        }
    }

    // partials [kvh][row < 8T][split][PART] of this wave's rows of present tokens (empty splits included: m = -inf,
    // l = 0, acc = 0, which the merge weighs 0)
    lsum += __shfl_xor(lsum, 32);
    const int t0 = tb + 4 * w;
    const size_t rbase = (size_t)kvh * T * GQA + (size_t)t0 * GQA;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int ri = 8 * (i >> 2) + 4 * h + (i & 3);
        if (t0 + (ri >> 3) < T) {
            float* pp = part + ((rbase + ri) * nch + c) * PART + PACC + r;
#pragma unroll
            for (int nb = 0; nb < 4; nb++) pp[32 * nb] = O[nb][i];
        }
    }
    if (h == 0 && t0 + (r >> 3) < T) {
        float* pp = part + ((rbase + r) * nch + c) * PART;
        pp[0] = m;
        pp[1] = lsum;
    }
}

// Merge of the splits with the sink (attn_fd_merge, flint_attn.wgsl:241-257): M = max(sink, m_c), out =
// sum_c 2^(m_c - M) acc_c / (2^(sink - M) + sum_c 2^(m_c - M) l_c), all in log2 units. Work-group = row (token, head);
// its 256 threads are 8 split lanes x 32 dim lanes (4 dims each): every split of the row is loaded in one round trip
// (split lane i takes splits i, i + 8, ...), then the split lanes are combined through LDS.
constexpr int MERGE_J = 16;  // splits per split lane: 8 x 16 >= the at most 128 splits of a plan

__global__ void __launch_bounds__(256) fl_merge(const float* __restrict__ part, int T, int nch,
                                                const float* __restrict__ sinks, float* __restrict__ out) {
    const int t = blockIdx.x / QH, head = blockIdx.x % QH, tid = threadIdx.x;
    const int cl = tid >> 5, d0 = (tid & 31) * 4;
    const float* p = part + ((size_t)(head / GQA) * T * GQA + (size_t)t * GQA + head % GQA) * nch * PART;
    __shared__ float red[8];
    __shared__ f32x4 accs[8][32];
    __shared__ float ls[8];
    float mj[MERGE_J], lj[MERGE_J];
    f32x4 aj[MERGE_J];
    float M = NEG_INF;
#pragma unroll
    for (int j = 0; j < MERGE_J; j++) {
        const int c = cl + 8 * j;
        mj[j] = NEG_INF;
        lj[j] = 0.f;
        aj[j] = f32x4{};
        if (c < nch) {
            const float* pc = p + (size_t)c * PART;
            mj[j] = pc[0];
            lj[j] = pc[1];
            aj[j] = *(const f32x4*)(pc + PACC + d0);
        }
        M = fmaxf(M, mj[j]);
    }
    if ((tid & 31) == 0) red[cl] = M;
    __syncthreads();
    M = sinks ? sinks[head] * LOG2E : NEG_INF;
#pragma unroll
    for (int i = 0; i < 8; i++) M = fmaxf(M, red[i]);
    f32x4 acc = f32x4{};
    float L = 0.f;
#pragma unroll
    for (int j = 0; j < MERGE_J; j++) {
        const float e = mj[j] == NEG_INF ? 0.f : exp2f(mj[j] - M);
        L += e * lj[j];
        acc += e * aj[j];
    }
    accs[cl][tid & 31] = acc;
    if ((tid & 31) == 0) ls[cl] = L;
    __syncthreads();
    if (tid < 32) {
        f32x4 sum = f32x4{};
        float lt = sinks && M != NEG_INF ? exp2f(sinks[head] * LOG2E - M) : 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            sum += accs[i][tid];
            lt += ls[i];
        }
        *(f32x4*)(out + ((size_t)t * QH + head) * HD + d0) = sum / lt;
    }
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

// NEOX RoPE: work-group (token, head), thread i rotates the pair (i, i + 64) (rope_neox_n, flint_attn.wgsl:46-53).
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


// ---- one or two tokens: 16 query rows (token * 8 + head) on the 16x16 f16 matrix units ----
// Work-group (key split, kv head), 4 waves; each wave owns whole 16-position subtiles (w, w + 4, ...) over all 128
// dims, so no per-tile exchange or barrier: S^T[16 keys][16 rows] is 4 dim steps of v_mfma_f32_16x16x32_f16 with
// A = K straight from HBM and B = Q (split into f16 hi + lo once, in registers), and P.V is 8 dim blocks of
// v_mfma_f32_16x16x16_f16 with A = P (split from the S^T registers: lane l holds row l % 16 and keys 4g + r,
// g = l / 16, register r) and B = V. f32 operands take three passes (hi.hi + hi.lo + lo.hi), an f16 cache's K or V
// two. The four waves' states are merged through LDS at the end; one partial per work-group.

template <int FMT>
struct SubRegs;
template <>
struct SubRegs<1> {  // f32: K dims 32a + 8g + 4e .. +3 of key l % 16 (index 2a + e); V keys 4g .. +3 of dim 16c + l % 16
    f32x4 k[8];
    f32x4 v[8];
};
template <>
struct SubRegs<0> {  // f16: K dims 32a + 8g .. +7 (a < 4); V keys 4g .. +3 of dim 16c + l % 16, 4 halves
    half8 k[4];
    half4 v[8];
};

template <int FMT, int NBUF>
__global__ void __launch_bounds__(256) fl_dec16(const void* __restrict__ kplane, const void* __restrict__ vplane,
                                                size_t plane_elems, int rows, const float* __restrict__ q, int T,
                                                int pos0, int win, float scale2, int klo, int span, int nch,
                                                float* __restrict__ part, unsigned* __restrict__ arrivals,
                                                const float* __restrict__ sinks, float* __restrict__ out) {
    constexpr int BPE = FMT == 1 ? 4 : 2;
    const int c = blockIdx.x % nch, kvh = blockIdx.x / nch;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, r16 = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: subtile addressing stays scalar
    const int lo_first = window_lo(pos0, win);
    const int cs = klo + chunk_lo(c, span, nch), ce = c + 1 < nch ? klo + chunk_lo(c + 1, span, nch) : klo + span;
    const int lo = max(cs, lo_first / TILE * TILE), hi = min(ce, pos0 + T);
    const int nsub = hi > lo ? (hi - lo + 15) / 16 : 0;

    const unsigned pbytes = (unsigned)(plane_elems * BPE);
    const rsrc_t kr = plane_rsrc((const char*)kplane + (size_t)kvh * plane_elems * BPE, pbytes);
    const rsrc_t vr = plane_rsrc((const char*)vplane + (size_t)kvh * plane_elems * BPE, pbytes);
    // the subtile's offset is wave-uniform and goes in the scalar operand; the lane offsets stay fixed, so the loop
    // writes no vector register for addresses (a pending load's destination is never reused for them)
    auto load = [&](SubRegs<FMT>& X, int j) {
        const int r0 = (lo + 16 * (j < nsub ? j : 0)) % rows;  // past the last: any subtile (never computed)
        const unsigned blk = (unsigned)(r0 / 32) * (32 * HD * BPE), sub = r0 % 32;
        const unsigned sk = __builtin_amdgcn_readfirstlane(blk + sub * 16);
        const unsigned sv = __builtin_amdgcn_readfirstlane(blk + (sub / (16 / BPE)) * HD * 16);
        if constexpr (FMT == 1) {
#pragma unroll
            for (int a = 0; a < 8; a++)
                X.k[a] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                    kr, ((8 * (a >> 1) + 2 * g + (a & 1)) * 32 + r16) * 16, sk, LOAD_NT));
#pragma unroll
            for (int cc = 0; cc < 8; cc++)
                X.v[cc] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        vr, (g * HD + 16 * cc + r16) * 16, sv, LOAD_NT));
        } else {
#pragma unroll
            for (int a = 0; a < 4; a++)
                X.k[a] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(
                                                       kr, ((4 * a + g) * 32 + r16) * 16, sk, LOAD_NT));
#pragma unroll
            for (int cc = 0; cc < 8; cc++)
                X.v[cc] = __builtin_bit_cast(half4, __builtin_amdgcn_raw_buffer_load_b64(
                                                        vr, ((g >> 1) * HD * 8 + (16 * cc + r16) * 8 + 4 * (g & 1)) * 2,
                                                        sv, 0));
        }
    };

    // the first subtiles' loads go out before Q's, so the two latencies overlap
    const int mine = nsub > w ? (nsub - w + 3) / 4 : 0;  // this wave's subtiles w, w + 4, ...
    SubRegs<FMT> R[NBUF];
#pragma unroll
    for (int k = 0; k < NBUF - 1; k++) load(R[k], w + 4 * k);
    __builtin_amdgcn_sched_barrier(0);

    // Q of the lane's row in registers, split into f16 hi + lo: step a holds dims 32a + 8g .. +7 (the B operand)
    half8 qh[4], ql[4];
    {
        const int t = r16 >> 3;
        const float* qr = q + ((size_t)t * QH + kvh * GQA + (r16 & 7)) * HD;
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const f32x4 x0 = t < T ? *(const f32x4*)(qr + 32 * a + 8 * g) : f32x4{};
            const f32x4 x1 = t < T ? *(const f32x4*)(qr + 32 * a + 8 * g + 4) : f32x4{};
            split8(x0, x1, qh[a], ql[a]);
        }
    }
    const int prow = pos0 + (r16 >> 3);
    const int plo = window_lo(prow, win);
    float m_run = NEG_INF, l_run = 0.f;
    f32x4 O[8];
#pragma unroll
    for (int cc = 0; cc < 8; cc++) O[cc] = f32x4{};
    auto step = [&](SubRegs<FMT>& X, int j) {
        const int k0 = lo + 16 * j;
        f32x4 S = f32x4{};
#pragma unroll
        for (int a = 0; a < 4; a++) {
            if constexpr (FMT == 1) {
                half8 kh, kl;
                split8(X.k[2 * a], X.k[2 * a + 1], kh, kl);
                S = mfma16k32(kh, qh[a], S);
                S = mfma16k32(kh, ql[a], S);
                S = mfma16k32(kl, qh[a], S);
            } else {
                S = mfma16k32(X.k[a], qh[a], S);
                S = mfma16k32(X.k[a], ql[a], S);
            }
        }
        float sv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int key = k0 + 4 * g + r;
            sv[r] = (key >= plo && key <= prow && key < hi) ? S[r] * scale2 : NEG_INF;
        }
        float mt = vmax3(vmax(sv[0], sv[1]), sv[2], sv[3]);  // masked scores are -inf, never NaN
        mt = vmax(mt, __shfl_xor(mt, 16));
        mt = max_xor32(mt);
        const float mn = fmaxf(m_run, mt);
        const float base = mn == NEG_INF ? 0.f : mn;
        const float cf = m_run == NEG_INF ? 0.f : fast_exp2(m_run - mn);
        float ls = 0.f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            sv[r] = fast_exp2(sv[r] - base);
            ls += sv[r];
        }
        ls += __shfl_xor(ls, 16);
        ls = add_xor32(ls);
        l_run = l_run * cf + ls;
        m_run = mn;
        if (__builtin_amdgcn_ballot_w64(cf != 1.f)) {  // register r of O holds row 4g + r
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float f = __shfl(cf, 4 * g + r);
#pragma unroll
                for (int cc = 0; cc < 8; cc++) O[cc][r] *= f;
            }
        }
        if (k0 < lo_first || k0 + 16 > hi) {  // rows of other or unwritten positions: no NaN through V
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int key = k0 + 4 * g + r;
                if (key < lo_first || key >= hi)
#pragma unroll
                    for (int cc = 0; cc < 8; cc++) {
                        if constexpr (FMT == 1) X.v[cc][r] = 0.f;
                        else X.v[cc][r] = (_Float16)0.f;
                    }
            }
        }
        half4 ph, pl;
        split4(f32x4{sv[0], sv[1], sv[2], sv[3]}, ph, pl);
#pragma unroll
        for (int cc = 0; cc < 8; cc++) {
            if constexpr (FMT == 1) {
                half4 vh, vl;
                split4(X.v[cc], vh, vl);
                O[cc] = mfma16k16(ph, vh, O[cc]);
                O[cc] = mfma16k16(ph, vl, O[cc]);
                O[cc] = mfma16k16(pl, vh, O[cc]);
            } else {
                O[cc] = mfma16k16(ph, X.v[cc], O[cc]);
                O[cc] = mfma16k16(pl, X.v[cc], O[cc]);
            }
        }
    };

    for (int i0 = 0; i0 < mine; i0 += NBUF) {
#pragma unroll
        for (int k = 0; k < NBUF; k++) {
            if (i0 + k < mine) {  // uniform in the wave
                load(R[(k + NBUF - 1) % NBUF], w + 4 * (i0 + k + NBUF - 1));
                __builtin_amdgcn_sched_barrier(0);  // the next subtile's loads issue before this one's wait
                step(R[k], w + 4 * (i0 + k));
            }
        }
    }

    // the four waves' states into one partial
    __shared__ f32x4 ob[4][8][64];
    __shared__ __attribute__((aligned(16))) float ml[4][2][16];
#pragma unroll
    for (int cc = 0; cc < 8; cc++) ob[w][cc][lane] = O[cc];
    if (g == 0) {
        ml[w][0][r16] = m_run;
        ml[w][1][r16] = l_run;
    }
    __syncthreads();
    // With the merge fused (arrivals != NULL, few splits), the partial is stored device-coherent (scope bit sc1,
    // through the XCD's L2) and the kv head's last work-group to arrive merges them all; no work-group waits.
    const bool fused = arrivals != nullptr;
    auto put = [&](float* p, float x) {
        if (fused) __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else *p = x;
    };
    const size_t rbase = (size_t)kvh * T * GQA;
    {
        // every wave combines dims 16cc .. 16cc + 15 of cc = 2w, 2w + 1 for its lane's rows 4g + r: the rows' factors
        // and the eight states read from LDS in one round, then the stores (no chain of dependent LDS reads)
        f32x4 mw[4], f[4], x[2][4];
#pragma unroll
        for (int ww = 0; ww < 4; ww++) mw[ww] = *(const f32x4*)&ml[ww][0][4 * g];
#pragma unroll
        for (int c2 = 0; c2 < 2; c2++)
#pragma unroll
            for (int ww = 0; ww < 4; ww++) x[c2][ww] = ob[ww][2 * w + c2][lane];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float M = NEG_INF;
#pragma unroll
            for (int ww = 0; ww < 4; ww++) M = fmaxf(M, mw[ww][r]);
#pragma unroll
            for (int ww = 0; ww < 4; ww++) f[ww][r] = mw[ww][r] == NEG_INF ? 0.f : exp2f(mw[ww][r] - M);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = 4 * g + r;
            if (row < T * GQA) {
                float* p = part + ((rbase + row) * nch + c) * PART + PACC + r16;
#pragma unroll
                for (int c2 = 0; c2 < 2; c2++) {
                    float o = 0.f;
#pragma unroll
                    for (int ww = 0; ww < 4; ww++) o += f[ww][r] * x[c2][ww][r];
                    put(p + 16 * (2 * w + c2), o);
                }
            }
        }
    }
    if (w == 0 && g == 0 && r16 < T * GQA) {
        float M = NEG_INF, Lt = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) M = fmaxf(M, ml[ww][0][r16]);
#pragma unroll
        for (int ww = 0; ww < 4; ww++)
            Lt += ml[ww][0][r16] == NEG_INF ? 0.f : exp2f(ml[ww][0][r16] - M) * ml[ww][1][r16];
        float* p = part + ((rbase + r16) * nch + c) * PART;
        put(p, M);
        put(p + 1, Lt);
    }
    if (!fused) return;
    // every wave's partial stores complete before the work-group barrier; wave 0 then releases at agent scope: the
    // partial happens before the arrival that counts it, and the kv head's last arrival acquires, so its merge reads
    // every partial
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ int last;
    if (w == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        int l = 0;
        if (lane == 0) {
            l = __hip_atomic_fetch_add(arrivals + kvh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                (unsigned)(nch - 1);
            if (l) __hip_atomic_store(arrivals + kvh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = l;
        }
        if (__builtin_amdgcn_readfirstlane(l)) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();  // the other waves see the acquiring wave's view through the work-group barrier
    if (!last) return;
    // the kv head's last work-group: the merge of fl_merge for its rows (row = token * 8 + head of the kv head, T * 8
    // <= 16), thread = (row, 8 dims), every split's partial loaded in one round trip (device-coherent loads)
    const int row = tid >> 4, d0 = (tid & 15) * 8;
    if (row >= T * GQA) return;
    const int head = kvh * GQA + (row & 7), t = row >> 3;
    const rsrc_t pr = plane_rsrc(part + (size_t)kvh * T * GQA * nch * PART, (unsigned)(T * GQA * nch * PART * 4));
    f32x4 hd[FL_FUSE_NCH], a0[FL_FUSE_NCH], a1[FL_FUSE_NCH];
#pragma unroll
    for (int cj = 0; cj < FL_FUSE_NCH; cj++) {
        const unsigned off = cj < nch ? (unsigned)(((row * nch + cj) * PART) * 4) : 0x7FFFFFF0u;
        const unsigned oa = off + (PACC + d0) * 4;
        hd[cj] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, off, 0, LOAD_SC1));
        a0[cj] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, oa, 0, LOAD_SC1));
        a1[cj] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, oa + 16, 0, LOAD_SC1));
    }
    const float sk = sinks ? sinks[head] * LOG2E : NEG_INF;
    float M = sk;
#pragma unroll
    for (int cj = 0; cj < FL_FUSE_NCH; cj++)
        if (cj < nch) M = fmaxf(M, hd[cj].x);
    f32x4 s0 = f32x4{}, s1 = f32x4{};
    float L = sinks && M != NEG_INF ? exp2f(sk - M) : 0.f;
#pragma unroll
    for (int cj = 0; cj < FL_FUSE_NCH; cj++) {
        const float e = cj < nch && hd[cj].x != NEG_INF ? exp2f(hd[cj].x - M) : 0.f;
        L += e * hd[cj].y;
        s0 += e * a0[cj];
        s1 += e * a1[cj];
    }
    float* o = out + ((size_t)t * QH + head) * HD + d0;
    *(f32x4*)o = s0 / L;
    *(f32x4*)(o + 4) = s1 / L;
}

// Merge for few splits (prefill blocks): 8 rows (token, head) per work-group of 256 threads, 4 dims per thread, the
// splits of a row loaded in one round trip.
constexpr int MERGE_FEW = 16;

template <int NJ>  // at most NJ splits
__global__ void __launch_bounds__(256) fl_merge_few(const float* __restrict__ part, int T, int nch,
                                                    const float* __restrict__ sinks, float* __restrict__ out) {
    const int rowid = blockIdx.x * 8 + (threadIdx.x >> 5);  // t * 32 + head
    if (rowid >= T * QH) return;
    const int t = rowid / QH, head = rowid % QH, d0 = (threadIdx.x & 31) * 4;
    const float* p = part + ((size_t)(head / GQA) * T * GQA + (size_t)t * GQA + head % GQA) * nch * PART;
    float mj[NJ], lj[NJ];
    f32x4 aj[NJ];
    float M = sinks ? sinks[head] * LOG2E : NEG_INF;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        mj[j] = NEG_INF;
        lj[j] = 0.f;
        aj[j] = f32x4{};
        if (j < nch) {
            const float* pc = p + (size_t)j * PART;
            mj[j] = pc[0];
            lj[j] = pc[1];
            aj[j] = *(const f32x4*)(pc + PACC + d0);
        }
        M = fmaxf(M, mj[j]);
    }
    float L = sinks && M != NEG_INF ? exp2f(sinks[head] * LOG2E - M) : 0.f;
    f32x4 acc = f32x4{};
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const float e = mj[j] == NEG_INF ? 0.f : exp2f(mj[j] - M);
        L += e * lj[j];
        acc += e * aj[j];
    }
    *(f32x4*)(out + ((size_t)t * QH + head) * HD + d0) = acc / L;
}

}  // namespace

Plan plan(int fmt, int pos0, int T, int win) {
    const int lo0 = win > 0 && pos0 + 1 > win ? pos0 + 1 - win : 0;
    const int klo = lo0 / 32 * 32, span = pos0 + T - klo;
    int nrb = (T + 3) / 4;
    int nch;
    int fused = 0;
    if (T <= 2 && span <= (fmt == 1 ? FL_FUSE_SPAN_F32 : FL_FUSE_SPAN_F16)) {  // fl_dec16 merging its own partials:
                                                                              // splits of at least FL_FUSE_SPLIT
        nch = span / FL_FUSE_SPLIT;
        nch = nch > FL_FUSE_NCH ? FL_FUSE_NCH : nch;
        fused = 1;
    } else if (T <= 2) {  // fl_dec16
        nch = span / FL_DEC_SPLIT;
        nch = nch > FL_DEC_NCH ? FL_DEC_NCH : nch;
    } else if (T <= 4) {  // one block of fl_attn: splits of at least 128 positions, 64 per kv head at most
        nch = span / 128;
        nch = nch > 64 ? 64 : nch;
    } else {  // fl_pf: blocks of 32 tokens, about one work-group per CU, splits of 64 positions or more, at most 64
        nrb = (T + PF_PT - 1) / PF_PT;
        nch = 256 / (nrb * KVH);
        const int most = span / 64, room = WS_ROWS / (T * GQA);
        nch = nch > most ? most : nch;
        nch = nch > room ? room : nch > 64 ? 64 : nch;
    }
    nch = nch < 1 ? 1 : nch;
    return Plan{klo, span, nch, nrb, fused};
}

size_t ws_floats() { return (size_t)KVH * WS_ROWS * PART + WS_ARRIVALS; }

hipError_t launch_attn(int fmt, const void* kp, const void* vp, int rows, const float* q, int T, int pos0, int win,
                       const Plan& p, float* ws, const float* sinks, float* out, hipStream_t st) {
    if ((size_t)T * GQA * p.nch > WS_ROWS) return hipErrorInvalidValue;  // the workspace's rows x splits per kv head
    const size_t pe = (size_t)rows * HD;
    const float scale2 = (1.0f / 11.313708498984761f) * LOG2E;  // 1/sqrt(128) (flint_attn.wgsl:92, 189) in log2 units
    const dim3 grid(p.nrb * p.nch * KVH);
    const Launch L{st};
    hipError_t e;
    // arrival counters of the fused decode merge, zero between launches, after the partials
    unsigned* arr = p.fused ? (unsigned*)(ws + (size_t)KVH * WS_ROWS * PART) : nullptr;
    if (p.fused && p.nch > FL_FUSE_NCH) return hipErrorInvalidValue;
    if (T <= 2) {  // decode (and 2-token steps): 16-row kernel
        e = fmt == 1 ? launch(fl_dec16<1, FL_DEC_BUF>, dim3(p.nch * KVH), dim3(256), L, kp, vp, pe, rows, q, T, pos0,
                              win, scale2, p.klo, p.span, p.nch, ws, arr, sinks, out)
                     : launch(fl_dec16<0, FL_DEC_BUF>, dim3(p.nch * KVH), dim3(256), L, kp, vp, pe, rows, q, T, pos0,
                              win, scale2, p.klo, p.span, p.nch, ws, arr, sinks, out);
        if (p.fused) return e;
    } else if (T <= 4) {  // one block of 4 tokens
        e = fmt == 1 ? launch(fl_attn<1, 2>, grid, dim3(256), L, kp, vp, pe, rows, q, T, pos0, win, scale2, p.klo,
                              p.span, p.nch, p.nrb, ws)
                     : launch(fl_attn<0, 2>, grid, dim3(256), L, kp, vp, pe, rows, q, T, pos0, win, scale2, p.klo,
                              p.span, p.nch, p.nrb, ws);
    } else {  // prefill: 32-token blocks over an LDS ring
        e = fmt == 1 ? launch(fl_pf<1>, grid, dim3(PF_NW * 64), L, kp, vp, pe, rows, q, T, pos0, win, scale2, p.klo,
                              p.span, p.nch, ws)
                     : launch(fl_pf<0>, grid, dim3(PF_NW * 64), L, kp, vp, pe, rows, q, T, pos0, win, scale2, p.klo,
                              p.span, p.nch, ws);
    }
    if (e != hipSuccess) return e;
    if (p.nch > 8 * MERGE_J) return hipErrorInvalidValue;
    // the smallest unrolled build that holds the plan's splits (each chunk slot is a predicated load)
    const dim3 g8((T * QH + 7) / 8);
    if (p.nch <= 4) return launch(fl_merge_few<4>, g8, dim3(256), L, (const float*)ws, T, p.nch, sinks, out);
    if (p.nch <= 8) return launch(fl_merge_few<8>, g8, dim3(256), L, (const float*)ws, T, p.nch, sinks, out);
    if (p.nch <= MERGE_FEW)
        return launch(fl_merge_few<MERGE_FEW>, g8, dim3(256), L, (const float*)ws, T, p.nch, sinks, out);
    return launch(fl_merge, dim3(T * QH), dim3(256), L, (const float*)ws, T, p.nch, sinks, out);
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
