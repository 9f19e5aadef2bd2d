// flint_store.cpp -- the Flint KV store and its C ABI (include/mechta_flint.h).
//
// Replaces the K/V buffers of Flint::new (flint.rs:227-232), the per-token uniforms (n, slot, lo, ring) that
// Flint::inputs writes for every layer (flint.rs:294-298) and the prefill block's (flint.rs:358-362), the root copies
// (read_root / write_root, flint.rs:320-331) and the ring photo (flint.rs:308-316).
#include <hip/hip_runtime.h>

#include <cmath>
#include <new>
#include <vector>

#include "../../include/mechta_flint.h"
#include "flint_internal.h"
#include "mkv_store.h"

using mkv::fail;
using mkv::hip_fail;
namespace fl = mkv::flint;

struct mfl_store {
    int layers = 0, ctx = 0, fmt = 0;
    std::vector<int> rows;       // per layer: 1024 (sliding) or ctx
    std::vector<unsigned char> swa;  // per layer: sliding window
    std::vector<size_t> off;     // per layer: byte offset of its first plane (K, kv head 0)
    char* base = nullptr;        // [layer][K|V][kv head] planes of rows x 128 elements
    size_t bytes = 0;
    float* ws = nullptr;         // split partials
    char* photo = nullptr;       // copies of the sliding layers' planes
    hipStream_t stream = nullptr;
};

namespace {

int bpe(const mfl_store* h) { return h->fmt == MKV_F16 ? 2 : 4; }
size_t plane_bytes(const mfl_store* h, int layer) { return (size_t)h->rows[layer] * fl::HD * bpe(h); }
char* plane(const mfl_store* h, int layer, int which) {
    return h->base + h->off[layer] + (size_t)which * fl::KVH * plane_bytes(h, layer);
}

int check(const mfl_store* h, int layer, const char* who) {
    if (!h) return fail(MKV_E_ARG, "%s: NULL handle", who);
    if (layer < 0 || layer >= h->layers) return fail(MKV_E_LAYER, "%s: layer %d outside [0, %d)", who, layer, h->layers);
    return MKV_OK;
}

}  // namespace

extern "C" {

int mfl_create(mfl_t** out, int layers, int ctx, int fmt, const unsigned char* sliding_mask, void* stream) {
    if (!out || !sliding_mask) return fail(MKV_E_ARG, "mfl_create: NULL argument");
    *out = nullptr;
    if (layers < 1) return fail(MKV_E_ARG, "mfl_create: %d layers", layers);
    if (fmt != MKV_F16 && fmt != MKV_F32) return fail(MKV_E_ARG, "mfl_create: format %d", fmt);
    if (ctx < 1024 || ctx > MKV_CTX_MAX || ctx % 1024)
        return fail(MKV_E_CTX, "mfl_create: context %d: must be a multiple of 1024 in [1024, %d]", ctx, MKV_CTX_MAX);
    mfl_store* h = new (std::nothrow) mfl_store;
    if (!h) return fail(MKV_E_NOMEM, "mfl_create: host allocation");
    h->layers = layers;
    h->ctx = ctx;
    h->fmt = fmt;
    h->stream = (hipStream_t)stream;
    size_t at = 0;
    for (int l = 0; l < layers; l++) {
        h->swa.push_back(sliding_mask[l] ? 1 : 0);
        h->rows.push_back(sliding_mask[l] ? MFL_RING_SWA : ctx);
        h->off.push_back(at);
        at += 2 * fl::KVH * plane_bytes(h, l);
    }
    h->bytes = at;
    hipError_t e = hipMalloc(&h->base, at);
    if (e == hipSuccess) e = hipMemsetAsync(h->base, 0, at, h->stream);
    if (e == hipSuccess) e = hipMalloc(&h->ws, fl::ws_floats() * sizeof(float));
    if (e == hipSuccess) e = hipMemsetAsync(h->ws, 0, fl::ws_floats() * sizeof(float), h->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        if (h->base) (void)hipFree(h->base);
        if (h->ws) (void)hipFree(h->ws);
        delete h;
        return fail(MKV_E_NOMEM, "mfl_create: %zu bytes of K/V: %s", at, hipGetErrorString(e));
    }
    *out = h;
    return MKV_OK;
}

int mfl_destroy(mfl_t* h) {
    if (!h) return MKV_OK;
    hipError_t e = hipStreamSynchronize(h->stream);
    if (h->base) (void)hipFree(h->base);
    if (h->ws) (void)hipFree(h->ws);
    if (h->photo) (void)hipFree(h->photo);
    delete h;
    return e == hipSuccess ? MKV_OK : hip_fail(e, "mfl_destroy");
}

int mfl_set_stream(mfl_t* h, void* stream) {
    if (!h) return fail(MKV_E_ARG, "mfl_set_stream: NULL handle");
    h->stream = (hipStream_t)stream;
    return MKV_OK;
}

int mfl_sync(mfl_t* h) {
    if (!h) return fail(MKV_E_ARG, "mfl_sync: NULL handle");
    hipError_t e = hipStreamSynchronize(h->stream);
    return e == hipSuccess ? MKV_OK : hip_fail(e, "mfl_sync");
}

int mfl_rows(const mfl_t* h, int layer, int* rows) {
    if (int rc = check(h, layer, "mfl_rows")) return rc;
    if (rows) *rows = h->rows[layer];
    return MKV_OK;
}

int mfl_rope_table(int pos, float base, float* tab) {
    if (!tab || pos < 0) return fail(MKV_E_ARG, "mfl_rope_table: bad argument");
    const float scale = powf(base, -2.0f / (float)fl::HD);
    float theta = (float)pos;
    for (int i = 0; i < fl::HD / 2; i++) {
        tab[i] = cosf(theta);
        tab[fl::HD / 2 + i] = sinf(theta);
        theta = theta * scale;
    }
    return MKV_OK;
}

int mfl_rope(mfl_t* h, int ntok, int heads, const float* x, const float* tab, float* out) {
    if (!h || !x || !tab || !out) return fail(MKV_E_ARG, "mfl_rope: NULL argument");
    if (ntok < 1 || heads < 1) return fail(MKV_E_ARG, "mfl_rope: %d tokens x %d heads", ntok, heads);
    hipError_t e = fl::launch_rope(ntok, heads, x, tab, out, h->stream);
    return e == hipSuccess ? MKV_OK : hip_fail(e, "mfl_rope");
}

int mfl_append(mfl_t* h, int layer, int pos0, int ntok, const float* k, const float* v) {
    if (int rc = check(h, layer, "mfl_append")) return rc;
    if (!k || !v) return fail(MKV_E_ARG, "mfl_append: NULL argument");
    const int rows = h->rows[layer];
    // a block of at most 512 tokens: on a sliding ring (1024 = 513 + 511 rows) it never overwrites a row that a
    // token of the same block still sees (flint.rs:24-26)
    if (ntok < 1 || ntok > MFL_BLOCK_MAX) return fail(MKV_E_ARG, "mfl_append: %d tokens outside [1, %d]", ntok,
                                                      MFL_BLOCK_MAX);
    if (pos0 < 0 || pos0 + ntok > h->ctx)
        return fail(MKV_E_POS, "mfl_append: positions [%d, %d) outside the context %d", pos0, pos0 + ntok, h->ctx);
    hipError_t e = fl::launch_append(h->fmt, plane(h, layer, 0), plane(h, layer, 1), rows, pos0, ntok, k, v,
                                     h->stream);
    return e == hipSuccess ? MKV_OK : hip_fail(e, "mfl_append");
}

int mfl_attend(mfl_t* h, int layer, int pos0, int ntok, const float* q, const float* sinks, float* out) {
    if (int rc = check(h, layer, "mfl_attend")) return rc;
    if (!q || !out) return fail(MKV_E_ARG, "mfl_attend: NULL argument");
    if (ntok < 1 || ntok > MFL_BLOCK_MAX) return fail(MKV_E_ARG, "mfl_attend: %d tokens outside [1, %d]", ntok,
                                                      MFL_BLOCK_MAX);
    if (pos0 < 0 || pos0 + ntok > h->ctx)
        return fail(MKV_E_POS, "mfl_attend: positions [%d, %d) outside the context %d", pos0, pos0 + ntok, h->ctx);
    const int rows = h->rows[layer];
    const int win = h->swa[layer] ? MFL_WINDOW : 0;
    const fl::Plan p = fl::plan(h->fmt, pos0, ntok, win);
    hipError_t e = fl::launch_attn(h->fmt, plane(h, layer, 0), plane(h, layer, 1), rows, q, ntok, pos0, win, p,
                                   h->ws, sinks, out, h->stream);
    return e == hipSuccess ? MKV_OK : hip_fail(e, "mfl_attend");
}

static int rows_io(mfl_t* h, int layer, int which, int r0, int r1, void* buf, int dir, const char* who) {
    if (int rc = check(h, layer, who)) return rc;
    if (which != MKV_K && which != MKV_V) return fail(MKV_E_ARG, "%s: which = %d", who, which);
    if (r0 < 0 || r1 < r0 || r1 > h->rows[layer]) return fail(MKV_E_POS, "%s: rows [%d, %d) of %d", who, r0, r1,
                                                             h->rows[layer]);
    if (!buf && r1 > r0) return fail(MKV_E_ARG, "%s: NULL buffer", who);
    hipError_t e = fl::launch_rows(h->fmt, plane(h, layer, which), h->rows[layer], which, r0, r1, buf, dir,
                                   h->stream);
    return e == hipSuccess ? MKV_OK : hip_fail(e, who);
}

int mfl_read_rows(mfl_t* h, int layer, int which, int r0, int r1, void* dst) {
    return rows_io(h, layer, which, r0, r1, dst, 0, "mfl_read_rows");
}

int mfl_write_rows(mfl_t* h, int layer, int which, int r0, int r1, const void* src) {
    return rows_io(h, layer, which, r0, r1, const_cast<void*>(src), 1, "mfl_write_rows");
}

static int photo_copy(mfl_t* h, bool take, const char* who) {
    if (!h) return fail(MKV_E_ARG, "%s: NULL handle", who);
    size_t need = 0;
    for (int l = 0; l < h->layers; l++)
        if (h->swa[l]) need += 2 * fl::KVH * plane_bytes(h, l);
    if (!take && !h->photo) return fail(MKV_E_ARG, "%s: no photo taken", who);
    hipError_t e = hipSuccess;
    if (!need) return fail(MKV_E_ARG, "%s: no sliding layer", who);
    if (take && !h->photo) {
        e = hipMalloc(&h->photo, need);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            h->photo = nullptr;
            return fail(MKV_E_NOMEM, "%s: %zu bytes", who, need);
        }
    }
    size_t at = 0;
    for (int l = 0; l < h->layers && e == hipSuccess; l++) {
        if (!h->swa[l]) continue;
        const size_t b = 2 * fl::KVH * plane_bytes(h, l);
        e = take ? hipMemcpyAsync(h->photo + at, h->base + h->off[l], b, hipMemcpyDeviceToDevice, h->stream)
                 : hipMemcpyAsync(h->base + h->off[l], h->photo + at, b, hipMemcpyDeviceToDevice, h->stream);
        at += b;
    }
    return e == hipSuccess ? MKV_OK : hip_fail(e, who);
}

int mfl_photo(mfl_t* h) { return photo_copy(h, true, "mfl_photo"); }
int mfl_restore_photo(mfl_t* h) { return photo_copy(h, false, "mfl_restore_photo"); }

}  // extern "C"
