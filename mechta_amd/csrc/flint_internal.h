// flint_internal.h -- geometry and launchers of the Flint KV path (flint_kv.hip, flint_store.cpp).
#pragma once
#include "mkv_internal.h"

namespace mkv {
namespace flint {

constexpr int KVH = 4;        // KV heads (flint.rs:14)
constexpr int QH = 32;        // query heads (flint.rs:13)
constexpr int HD = 128;       // head_dim (flint.rs:15)
constexpr int GQA = QH / KVH;
constexpr int PART = 4 + HD;  // split partial: [m, l, 0, 0, acc[128]]
constexpr int PACC = 4;

// Element offsets of (row, d) inside one plane of a kv head. f32: K [row/32][d/4][row%32][4], V [row/4][d][row%4];
// f16: K [row/32][d/8][row%32][8], V [row/8][d][row%8].
__host__ __device__ inline size_t k_off(int r, int d) {
    return (size_t)(r / 32) * (32 * HD) + (size_t)(d / 4) * (32 * 4) + (size_t)(r % 32) * 4 + (d % 4);
}
__host__ __device__ inline size_t v_off32(int r, int d) {
    return (size_t)(r / 4) * (4 * HD) + (size_t)d * 4 + (r % 4);
}
__host__ __device__ inline size_t k_off16(int r, int d) {
    return (size_t)(r / 32) * (32 * HD) + (size_t)(d / 8) * (32 * 8) + (size_t)(r % 32) * 8 + (d % 8);
}
__host__ __device__ inline size_t v_off16(int r, int d) {
    return (size_t)(r / 8) * (8 * HD) + (size_t)d * 8 + (r % 8);
}

// Splits of one attention call: keys [klo, klo + span) (klo = the first token's window start rounded down to 32),
// nch splits at chunk_lo boundaries, nrb token blocks (4 tokens; 32 for a prefill of more than 4); fused: a decode
// whose kernel merges its own few splits (no merge launch).
struct Plan {
    int klo, span, nch, nrb, fused;
};
constexpr int WS_ROWS = 16384;  // rows x splits per kv head that the split partials hold
constexpr int WS_ARRIVALS = 64;  // floats after the partials: the fused decode's arrival counters (zero at creation)
Plan plan(int fmt, int pos0, int T, int win);
size_t ws_floats();  // split partials of any plan (4 kv heads x WS_ROWS x PART) and the arrival counters

hipError_t launch_attn(int fmt, const void* kp, const void* vp, int rows, const float* q, int T, int pos0, int win,
                       const Plan& p, float* ws, const float* sinks, float* out, hipStream_t st);
hipError_t launch_append(int fmt, void* kp, void* vp, int rows, int pos0, int ntok, const float* k, const float* v,
                         hipStream_t st);
hipError_t launch_rope(int ntok, int heads, const float* x, const float* tab, float* out, hipStream_t st);
hipError_t launch_rows(int fmt, void* plane, int rows, int which, int r0, int r1, void* buf, int dir, hipStream_t st);

}  // namespace flint
}  // namespace mkv
