// mkv_internal.h -- shared definitions of libmechta_kv: store layout, launch helper, kernel launchers.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <tuple>

namespace mkv {

constexpr int KVH = 2;       // KV heads
constexpr int QH = 16;       // query heads (GQA 8:1)
constexpr int HD = 256;      // head_dim
constexpr int GQA = QH / KVH;
constexpr int KBLK = 32;     // K plane: positions per block, [pos/32][d/8][pos%32][8]
constexpr int VGRP = 8;      // V plane: positions per group, [pos/8][d][pos%8]
constexpr int VGRP32 = 4;    // f32 V plane: positions per group, [pos/4][d][pos%4]
constexpr int NXCD = 8;      // accelerator dies (XCDs) of the MI355X, each with its own L2
constexpr int ROWS = 32;     // query rows per KV head in decode: 4 tokens x 8 heads
constexpr int PART = 4 + HD; // split-K partial: [m, l, 0, 0, acc[256]] (acc 16-byte aligned)
constexpr int PACC = 4;      // offset of acc in a partial
constexpr size_t STORE_SLACK = 64 * HD * 4;  // bytes allocated past the last plane (see mkv_create)

// Element offset of (pos, d) inside one f16 K plane.
__host__ __device__ inline size_t k_off(int pos, int d) {
    return (size_t)(pos / KBLK) * (KBLK * HD) + (size_t)(d / 8) * (KBLK * 8) + (size_t)(pos % KBLK) * 8 + (d % 8);
}
// Element offset of (pos, d) inside one f16 V plane.
__host__ __device__ inline size_t v_off(int pos, int d) {
    return (size_t)(pos / VGRP) * (VGRP * HD) + (size_t)d * VGRP + (pos % VGRP);
}

// Element offset of (pos, d) inside one f32 K plane: [pos/32][d/4][pos%32][4].
__host__ __device__ inline size_t k_off32(int pos, int d) {
    return (size_t)(pos / KBLK) * (KBLK * HD) + (size_t)(d / 4) * (KBLK * 4) + (size_t)(pos % KBLK) * 4 + (d % 4);
}
// Element offset of (pos, d) inside one f32 V plane: [pos/4][d][pos%4].
__host__ __device__ inline size_t v_off32(int pos, int d) {
    return (size_t)(pos / VGRP32) * (VGRP32 * HD) + (size_t)d * VGRP32 + (pos % VGRP32);
}
// Positions per layout unit of a plane: K blocks of 32 in both formats, V groups of 8 (f16) or 4 (f32).
__host__ __device__ inline int plane_unit(int fmt, int which) { return which == 0 ? KBLK : fmt == 0 ? VGRP : VGRP32; }

// f32 -> f16 bits: v_cvt_f16_f32 rounds to nearest even and keeps subnormals.
__device__ inline unsigned short f2h(float x) {
    _Float16 h = (_Float16)x;
    return __builtin_bit_cast(unsigned short, h);
}

// NEOX RoPE value of dim d of one 256-dim K row a, table tb = [cos 0..31 | sin 0..31] (kv_src, kv.wgsl:19-23):
// d < 32: a[d]c[d] - a[d+32]s[d]; 32 <= d < 64 (i = d - 32): a[i]s[i] + a[d]c[i]; else a[d].
// Every product and the sum are rounded to f32 separately (no FMA contraction).
__device__ inline float rope_dim(const float* __restrict__ a, const float* __restrict__ tb, int d) {
#pragma clang fp contract(off)
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

// Split-K chunks: chunk c (of nch) starts at chunk_lo(c) = c * span / nch rounded down to a whole 32-position K block;
// the last chunk ends where the keys end (span may exceed them: the last chunk is then shorter than the others).
__host__ __device__ inline int chunk_lo(int c, int span, int nch) {
    return (int)((long long)c * span / nch / KBLK * KBLK);
}
// Chunks [c0, c1) are the ones holding a position of [lo, hi) (lo < hi <= the keys' end). span == 0 marks an
// interleaved split (each split holds positions spread over the whole range): every split is a candidate.
__host__ __device__ inline void chunk_range(int lo, int hi, int span, int nch, int& c0, int& c1) {
    if (span == 0) {
        c0 = 0;
        c1 = nch;
        return;
    }
    c0 = (int)((long long)lo * nch / span);  // estimates, then exact by the boundaries
    while (c0 > 0 && chunk_lo(c0, span, nch) > lo) c0--;
    while (c0 + 1 < nch && chunk_lo(c0 + 1, span, nch) <= lo) c0++;
    c1 = (int)((long long)hi * nch / span);
    while (c1 > 0 && chunk_lo(c1, span, nch) >= hi) c1--;
    while (c1 < nch && chunk_lo(c1, span, nch) < hi) c1++;
}

// Geometry of one store, passed by value to launchers.
struct Geom {
    int layers, ctx, fmt;  // fmt: 0 = f16, 1 = f32
    size_t plane_elems;    // ctx * 256
    int bpe() const { return fmt == 0 ? 2 : 4; }
    size_t plane_bytes() const { return plane_elems * (size_t)bpe(); }
    // plane index of (layer, which, kvh): [layer][K|V][kvh]
    size_t plane(int layer, int which, int kvh) const { return ((size_t)layer * 2 + which) * KVH + kvh; }
};

// Where and how a kernel is launched: the stream, and two events that (when set) take the kernel's start and end
// timestamps from its dispatch packet (hipExtLaunchKernel), so traced kernel times are the kernels' own durations.
struct Launch {
    hipStream_t s;
    hipEvent_t a = nullptr, b = nullptr;
};

template <typename... P, typename... A>
hipError_t launch(void (*k)(P...), dim3 grid, dim3 block, const Launch& L, A... a) {
    static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
    std::tuple<P...> t{static_cast<P>(a)...};
    void* args[sizeof...(P) > 0 ? sizeof...(P) : 1];
    std::apply([&](auto&... x) {
        int i = 0;
        ((args[i++] = (void*)&x), ...);
    }, t);
    return hipExtLaunchKernel((const void*)k, grid, block, args, 0, L.s, L.a, L.b, 0);
}

// Decode workspace: partials of the split-K decode.
struct DecodeWs {
    float* part;      // [KVH*ROWS][max_chunks][PART]
    int max_chunks;
};

// Rows appended by the decode kernel itself (mkv_append_decode): ntok = 0 for none.
struct FusedAppend {
    const float* kn = nullptr;  // [ntok][2][256]
    const float* v = nullptr;   // [ntok][512]
    const float* tab = nullptr; // [ntok][64]
    int pos = 0, ntok = 0;
};

// ---- launchers (kernels live in kv_append.hip, kv_decode.hip, kv_prefill.hip) ----
hipError_t launch_append(const Geom& g, void* base, int layer, int pos, int ntok, const float* kn, const float* v,
                         const float* tab, const Launch& L);
hipError_t launch_read_rows(const Geom& g, const void* base, int layer, int which, int p0, int p1, void* dst,
                            const Launch& L);
hipError_t launch_write_rows(const Geom& g, void* base, int layer, int which, int p0, int p1, const void* src,
                             const Launch& L);
// Split-K pass and merge of the decode on the f16 store (two kernels): span = 0, c0 = 0 and the keys [s0, kend) are nu stages of KPS_F16 positions (s0 = start rounded down to
// a stage), dealt round robin to nch work-groups, the partial round first.
constexpr int KPS_F16 = 64;
struct DecodePlan {
    int span, nch, c0, s0, nu;
};
DecodePlan decode_plan(int n, int ntok, int start);
hipError_t launch_decode_core(const Geom& g, void* base, int layer, const float* q, int ntok, int n, int start,
                              float scale, const DecodePlan& p, const DecodeWs& ws, const FusedAppend& fa,
                              const Launch& L);
hipError_t launch_decode_merge(int ntok, int n, int start, const DecodePlan& p, const DecodeWs& ws, const float* gate,
                               void* out, bool h16, const Launch& L);
// Small prefill blocks on the f16 store (T < SMALL_PREFILL_MAX): the reference runs them through attn_fd4 (f32 Q,
// exact f32 softmax; engine.rs:1237-1241), so they run on decode_f16's f32-class arithmetic, one column of work-groups
// per block of 4 tokens over the decode's stages; partials [kvh][row < 32 nzb][nch][PART], then launch_merge.
constexpr int SMALL_PREFILL_MAX = 63;
struct SmallPlan {
    DecodePlan d;
    int nzb;  // blocks of 4 tokens
};
SmallPlan small_prefill_plan(int T, int n, int start);
size_t small_prefill_ws_floats(int T, int nch);
hipError_t launch_small_prefill(const Geom& g, const void* base, int layer, const float* q, int T, int n, int start,
                                float scale, const SmallPlan& p, float* ws, const Launch& L);
// Merge of split-K partials laid out [kvh][row < rpk][chunk < nch][PART], row = token*8 + head of the kv head:
// out[t][head] for t < ntok over the chunks (chunk_lo of span, nch) holding a key of [start, n + t), optional gate;
// out is f32, or with h16 f16 bits rounded to nearest even (attn_gate16).
hipError_t launch_merge(const float* part, int rpk, int ntok, int n, int start, int span, int nch, const float* gate,
                        void* out, bool h16, const Launch& L);
// q/k producer (rmsnorm of the q and k heads, rope2 of q) of ntok tokens; tab: [ntok][64] device RoPE rows.
hipError_t launch_qk_produce(int ntok, const float* qf, const float* kb, const float* q_w, const float* k_w,
                             float eps, const float* tab, float* q_out, float* kn_out, const Launch& L);
// Decode attention over the f32 store (kv_attn32.hip, T <= 4): one block of 4 tokens (nrb = 1, c0 = 0), nch
// work-groups per kv head taking the window's 32-key tiles round robin (span 0); partials [kvh][row < rpk][nch][PART],
// then launch_merge.
struct Attn32Plan {
    int span, nch, c0, nrb;
};
Attn32Plan attn32_plan(int T, int n, int start);
hipError_t launch_attn_f32(const Geom& g, const void* base, int layer, const float* q, int T, int n, int start,
                           float scale, const Attn32Plan& p, int rpk, float* part, const FusedAppend& fa,
                           const Launch& L);
// Prefill: split-K pass into the partials ws, then launch_merge with the returned plan.
struct PrefillPlan {
    int span, nch;  // splits of [0, span) as chunk_lo
};
PrefillPlan prefill_plan(int T, int n);
size_t prefill_ws_floats(int T, int nch);
hipError_t launch_prefill(const Geom& g, const void* base, int layer, const float* q, int T, int n, int start,
                          float scale, const PrefillPlan& p, float* ws, const Launch& L);
// f32 store: prefill_f32 (16-token work-groups over an LDS ring, f32-class arithmetic)
PrefillPlan prefill32_plan(int T, int n);
hipError_t launch_prefill_f32(const Geom& g, const void* base, int layer, const float* q, int T, int n, int start,
                              float scale, const PrefillPlan& p, float* ws, const Launch& L);

}  // namespace mkv
