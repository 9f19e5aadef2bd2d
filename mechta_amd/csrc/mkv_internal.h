// mkv_internal.h -- shared definitions of libmechta_kv: store layout, kernel launchers, error plumbing.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

namespace mkv {

constexpr int KVH = 2;       // KV heads
constexpr int QH = 16;       // query heads (GQA 8:1)
constexpr int HD = 256;      // head_dim
constexpr int GQA = QH / KVH;
constexpr int KBLK = 32;     // K plane: positions per block, [pos/32][d/8][pos%32][8]
constexpr int VGRP = 8;      // V plane: positions per group, [pos/8][d][pos%8]
constexpr int ROWS = 32;     // query rows per KV head in decode: 4 tokens x 8 heads
constexpr int PART = 2 + HD; // split-K partial: [m, l, acc[256]]

// Element offset of (pos, d) inside one f16 K plane.
__host__ __device__ inline size_t k_off(int pos, int d) {
    return (size_t)(pos / KBLK) * (KBLK * HD) + (size_t)(d / 8) * (KBLK * 8) + (size_t)(pos % KBLK) * 8 + (d % 8);
}
// Element offset of (pos, d) inside one f16 V plane.
__host__ __device__ inline size_t v_off(int pos, int d) {
    return (size_t)(pos / VGRP) * (VGRP * HD) + (size_t)d * VGRP + (pos % VGRP);
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

// Decode workspace: partials of the split-K decode.
struct DecodeWs {
    float* part;      // [KVH*ROWS][max_chunks][PART]
    int max_chunks;
};

// ---- launchers (kernels live in kv_append.hip, kv_decode.hip, kv_prefill.hip) ----
hipError_t launch_append(const Geom& g, void* base, int layer, int pos, int ntok, const float* kn, const float* v,
                         const float* tab, hipStream_t s);
hipError_t launch_read_rows(const Geom& g, const void* base, int layer, int which, int p0, int p1, void* dst,
                            hipStream_t s);
hipError_t launch_write_rows(const Geom& g, void* base, int layer, int which, int p0, int p1, const void* src,
                             hipStream_t s);
// Split-K pass and merge of the decode (two kernels, both on stream s).
struct DecodePlan {
    int ch, nch, c0;
};
DecodePlan decode_plan(int n, int ntok, int start);
hipError_t launch_decode_core(const Geom& g, const void* base, int layer, const float* q, int ntok, int n, int start,
                              float scale, const DecodePlan& p, const DecodeWs& ws, hipStream_t s);
hipError_t launch_decode_merge(int ntok, int n, int start, const DecodePlan& p, const DecodeWs& ws, const float* gate,
                               float* out, hipStream_t s);
hipError_t launch_prefill(const Geom& g, const void* base, int layer, const float* q, int T, int n, int start,
                          float scale, float* out, const float* gate, float* ws, size_t ws_floats, hipStream_t s);
size_t prefill_ws_floats(int ctx);

}  // namespace mkv
