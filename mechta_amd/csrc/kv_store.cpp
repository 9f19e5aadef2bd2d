// kv_store.cpp -- the KV store object and the C ABI of libmechta_kv (declared in include/mechta_kv.h).
//
// The store replaces the reference's per-layer K/V wgpu buffers (engine.rs:493-496) and the host side of the
// dispatches that touch them (uniform writes engine.rs:618-673, quad.rs:277-289, engine.rs:902-931; root I/O
// engine.rs:782-823). Argument checks return the error codes of the header where the reference panics.
#include <algorithm>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/mechta_kv.h"
#include "mkv_internal.h"
#include "mkv_store.h"

using namespace mkv;

namespace mkv {
thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what) { return fail(MKV_E_HIP, "%s: %s", what, hipGetErrorString(e)); }
}  // namespace mkv

namespace {

using mkv::fail;
using mkv::hip_fail;

// Scratch of mkv_append_decode_noalloc: the split-K partials of one decode (2 kv heads x 32 rows x up to 248 splits x
// 260 floats = 16,506,880 bytes), a file-scope device array instead of the handle's workspace, so that the call
// allocates nothing. Each GPU holds its own copy until the process ends. Host code never uses the array's name as a
// device address: its per-device address comes from hipGetSymbolAddress, resolved once per device with that device
// current, by mkv_create (whose other work does not depend on it) or else by the entry point's first call there. Every call on one GPU shares it; calls that overlap on one GPU (other streams, other
// handles) race. No part needs clearing: a decode reads only partials its own core launch wrote.
constexpr int SCRATCH_CHUNKS = 248;
constexpr size_t SCRATCH_FLOATS = (size_t)KVH * ROWS * SCRATCH_CHUNKS * PART;
static __device__ __align__(256) float scratch[SCRATCH_FLOATS];
constexpr int MAX_DEVICES = 64;
float* g_scratch[MAX_DEVICES] = {};
std::mutex g_scratch_mu;

// Resolves (once) the scratch's address on `dev`, the current device.
hipError_t resolve_scratch(int dev) {
    if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch[dev]) return hipSuccess;
    float* p = nullptr;
    hipError_t e = hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch[dev] = p;
    return hipSuccess;
}

float* scratch_of(int dev) {
    if (dev < 0 || dev >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return g_scratch[dev];
}

int check_layer(const mkv_store* h, int layer) {
    if (layer < 0 || layer >= h->g.layers) return fail(MKV_E_LAYER, "layer %d outside [0, %d)", layer, h->g.layers);
    return MKV_OK;
}

constexpr size_t TRACE_RESERVE = 1024;  // events mkv_trace keeps ready: two per traced launch

hipEvent_t take_event(mkv_store* h) {
    if (!h->pool.empty()) {
        hipEvent_t e = h->pool.back();
        h->pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Runs `fn(const Launch&)`, which enqueues one kernel on h->stream; while tracing, the kernel's own start and end
// timestamps land in two events kept for mkv_trace_read.
template <typename F>
hipError_t traced(mkv_store* h, int kind, F&& fn) {
    Launch L{h->stream};
    if (!h->tracing) return fn(L);
    L.a = take_event(h);
    L.b = take_event(h);
    if (!L.a || !L.b) return hipErrorOutOfMemory;
    hipError_t e = fn(L);
    if (e == hipSuccess) {
        h->pending.push_back({kind, L.a, L.b});
    } else {
        h->pool.push_back(L.a);
        h->pool.push_back(L.b);
    }
    return e;
}

// out: f32, or f16 bits (h16, attn_gate16's output)
hipError_t decode_all(mkv_store* h, const DecodeWs& ws, int layer, const float* q, int ntok, int n, int start,
                      float scale, void* out, bool h16, const float* gate, const FusedAppend& fa = FusedAppend{}) {
    if (h->g.fmt == MKV_F32) {
        const Attn32Plan p = attn32_plan(ntok, n, start);
        if (p.nch > ws.max_chunks) return hipErrorInvalidValue;
        hipError_t e = traced(h, MKV_SPAN_CORE, [&](const Launch& L) {
            return launch_attn_f32(h->g, h->base, layer, q, ntok, n, start, scale, p, ROWS, ws.part, fa, L);
        });
        if (e != hipSuccess) return e;
        return traced(h, MKV_SPAN_MERGE, [&](const Launch& L) {
            return launch_merge(ws.part, ROWS, ntok, n, start, p.span, p.nch, gate, out, h16, L);
        });
    }
    DecodePlan p = decode_plan(n, ntok, start);
    hipError_t e = traced(h, MKV_SPAN_CORE, [&](const Launch& L) {
        return launch_decode_core(h->g, h->base, layer, q, ntok, n, start, scale, p, ws, fa, L);
    });
    if (e != hipSuccess) return e;
    return traced(h, MKV_SPAN_MERGE,
                  [&](const Launch& L) { return launch_decode_merge(ntok, n, start, p, ws, gate, out, h16, L); });
}

// Floats of the prefill partials workspace, allocated with the store: the largest any prefill plan uses (the f16
// plans keep T * splits <= 4096, the f32 plan <= 2048, the small-block plan <= 4096 rows per kv head).
size_t prefill_ws_max_floats() {
    size_t m = 0;
    for (int T = 1; T <= MKV_PREFILL_MAX; T++) {
        for (int n : {1, 64, 1024, 8192, MKV_CTX_MAX - T}) {
            m = std::max(m, prefill_ws_floats(T, prefill_plan(T, n).nch));
            m = std::max(m, prefill_ws_floats(T, prefill32_plan(T, n).nch));
            if (T <= SMALL_PREFILL_MAX) m = std::max(m, small_prefill_ws_floats(T, small_prefill_plan(T, n, 0).d.nch));
        }
    }
    return m;
}

void free_events(mkv_store* h) {
    for (auto& s : h->pending) {
        (void)hipEventDestroy(s.a);
        (void)hipEventDestroy(s.b);
    }
    for (auto e : h->pool) (void)hipEventDestroy(e);
    h->pending.clear();
    h->pool.clear();
}

// Device bytes of one store: the planes (layers x {K, V} x 2 heads x ctx x 256 elements: exactly the reference's
// 2 x layers KV buffers of buffer_bytes_for(ctx), engine.rs:64-65) plus the slack past the last plane, then the decode
// partials (2 kv heads x 32 rows x splits x 260 floats) and the prefill partials (prefill_ws_max_floats).
struct StoreBytes {
    size_t planes, slack, decode_ws, prefill_ws;
    int max_chunks;
    size_t total() const { return planes + slack + decode_ws + prefill_ws; }
};
StoreBytes store_bytes(int layers, int ctx, int fmt) {
    StoreBytes b;
    b.planes = (size_t)layers * 2 * KVH * (size_t)ctx * HD * (fmt == MKV_F16 ? 2 : 4);
    b.slack = STORE_SLACK;
    // decode splits: f16 one per 64-position stage, at most 108 (small prefill blocks 124); f32 at most 248
    b.max_chunks = std::min(ctx / 64 + 2, 256);
    b.decode_ws = (size_t)KVH * ROWS * b.max_chunks * PART * sizeof(float);
    b.prefill_ws = prefill_ws_max_floats() * sizeof(float);
    return b;
}

}  // namespace

extern "C" {

const char* mkv_last_error(void) { return g_err; }

size_t mkv_buffer_bytes(int ctx, int fmt) {
    if (ctx < 0 || (fmt != MKV_F16 && fmt != MKV_F32)) return 0;
    return (size_t)ctx * (KVH * HD) * (fmt == MKV_F16 ? 2 : 4);
}

size_t mkv_store_bytes(int layers, int ctx, int fmt) {
    if (layers < 1 || layers > 4096 || (fmt != MKV_F16 && fmt != MKV_F32) || ctx % 1024 != 0 || ctx < MKV_CTX_MIN ||
        ctx > MKV_CTX_MAX)
        return 0;
    return store_bytes(layers, ctx, fmt).total();
}

int mkv_create(mkv_t** out, int layers, int ctx, int fmt, void* stream) {
    if (!out) return fail(MKV_E_ARG, "mkv_create: out is NULL");
    *out = nullptr;
    if (layers < 1 || layers > 4096) return fail(MKV_E_ARG, "mkv_create: layers %d", layers);
    if (fmt != MKV_F16 && fmt != MKV_F32) return fail(MKV_E_ARG, "mkv_create: format %d (use MKV_F16 or MKV_F32)", fmt);
    if (ctx % 1024 != 0 || ctx < MKV_CTX_MIN || ctx > MKV_CTX_MAX)
        return fail(MKV_E_CTX, "context %d: must be a multiple of 1024 between %d and %d", ctx, MKV_CTX_MIN,
                    MKV_CTX_MAX);
    int dev = 0;
    hipError_t de = hipGetDevice(&dev);
    if (de != hipSuccess) return hip_fail(de, "mkv_create: current device");
    // the no-allocation entry point's scratch address on this device, resolved here while the device is current; a
    // failure leaves that one entry point unavailable on the device (it then returns MKV_E_HIP), nothing else
    (void)resolve_scratch(dev);
    mkv_store* h = new (std::nothrow) mkv_store;
    if (!h) return fail(MKV_E_NOMEM, "mkv_create: host allocation");
    h->device = dev;
    h->g.layers = layers;
    h->g.ctx = ctx;
    h->g.fmt = fmt;
    h->g.plane_elems = (size_t)ctx * HD;
    h->stream = (hipStream_t)stream;
    h->len.assign(layers, 0);
    // + slack: a decode stage starting on a 32-position boundary reads up to 64 positions, which may reach past the
    // last plane's end (the rows read there are masked, never used)
    const StoreBytes sb = store_bytes(layers, ctx, fmt);
    size_t bytes = sb.planes + sb.slack;
    hipError_t e = hipMalloc(&h->base, bytes);
    if (e != hipSuccess) {
        delete h;
        (void)hipGetLastError();
        return fail(MKV_E_NOMEM, "mkv_create: hipMalloc of %zu bytes failed", bytes);
    }
    h->dws.max_chunks = sb.max_chunks;
    e = hipMalloc(&h->dws.part, sb.decode_ws);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(h->base);
        if (h->dws.part) (void)hipFree(h->dws.part);
        delete h;
        return fail(MKV_E_NOMEM, "mkv_create: workspace allocation failed");
    }
    h->pws_floats = sb.prefill_ws / sizeof(float);
    e = hipMalloc(&h->pws, h->pws_floats * sizeof(float));
    if (e != hipSuccess) {
        const size_t pbytes = h->pws_floats * sizeof(float);
        (void)hipGetLastError();
        (void)hipFree(h->base);
        (void)hipFree(h->dws.part);
        delete h;
        return fail(MKV_E_NOMEM, "mkv_create: prefill workspace allocation (%zu bytes) failed", pbytes);
    }
    // zero fill: positions never written read as 0 (wgpu zero-initialises the reference's buffers)
    e = hipMemsetAsync(h->base, 0, bytes, h->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
    if (e != hipSuccess) {
        int rc = hip_fail(e, "mkv_create: zero fill");
        (void)hipFree(h->base);
        (void)hipFree(h->dws.part);
        if (h->pws) (void)hipFree(h->pws);
        delete h;
        return rc;
    }
    *out = h;
    return MKV_OK;
}

int mkv_destroy(mkv_t* h) {
    if (!h) return MKV_OK;
    root_free(h);
    hipError_t e = hipStreamSynchronize(h->stream);
    free_events(h);
    (void)hipFree(h->base);
    (void)hipFree(h->dws.part);
    if (h->pws) (void)hipFree(h->pws);
    if (h->rope_dev) (void)hipFree(h->rope_dev);
    delete h;
    return e == hipSuccess ? MKV_OK : hip_fail(e, "mkv_destroy");
}

int mkv_set_stream(mkv_t* h, void* stream) {
    if (!h) return fail(MKV_E_ARG, "mkv_set_stream: NULL handle");
    h->stream = (hipStream_t)stream;
    return MKV_OK;
}

int mkv_sync(mkv_t* h) {
    if (!h) return fail(MKV_E_ARG, "mkv_sync: NULL handle");
    hipError_t e = hipStreamSynchronize(h->stream);
    return e == hipSuccess ? MKV_OK : hip_fail(e, "mkv_sync");
}

int mkv_info(const mkv_t* h, int* layers, int* ctx, int* fmt) {
    if (!h) return fail(MKV_E_ARG, "mkv_info: NULL handle");
    if (layers) *layers = h->g.layers;
    if (ctx) *ctx = h->g.ctx;
    if (fmt) *fmt = h->g.fmt;
    return MKV_OK;
}

int mkv_len(const mkv_t* h, int layer, int* len) {
    if (!h || !len) return fail(MKV_E_ARG, "mkv_len: NULL argument");
    if (int rc = check_layer(h, layer)) return rc;
    *len = h->len[layer];
    return MKV_OK;
}

int mkv_append(mkv_t* h, int layer, int pos, int ntok, const float* kn, const float* v, const float* tab) {
    if (!h || !kn || !v || !tab) return fail(MKV_E_ARG, "mkv_append: NULL argument");
    if (int rc = check_layer(h, layer)) return rc;
    if (ntok < 1 || ntok > MKV_PREFILL_MAX) return fail(MKV_E_ARG, "mkv_append: ntok %d outside [1, %d]", ntok,
                                                        MKV_PREFILL_MAX);
    if (pos < 0 || pos + ntok > h->g.ctx)
        return fail(MKV_E_POS, "mkv_append: positions [%d, %d) outside the context %d", pos, pos + ntok, h->g.ctx);
    if (pos > h->len[layer])
        return fail(MKV_E_POS, "mkv_append: position %d leaves a hole after the written length %d", pos,
                    h->len[layer]);
    hipError_t e = traced(h, MKV_SPAN_KV_WRITE, [&](const Launch& L) {
        return launch_append(h->g, h->base, layer, pos, ntok, kn, v, tab, L);
    });
    if (e != hipSuccess) return hip_fail(e, "mkv_append");
    h->len[layer] = pos + ntok;
    return MKV_OK;
}

int mkv_set_len(mkv_t* h, int len) {
    if (!h) return fail(MKV_E_ARG, "mkv_set_len: NULL handle");
    for (int l = 0; l < h->g.layers; l++)
        if (len < 0 || len > h->len[l])
            return fail(MKV_E_POS, "mkv_set_len: %d is past the written length %d of layer %d", len, h->len[l], l);
    for (int l = 0; l < h->g.layers; l++) h->len[l] = len;
    return MKV_OK;
}

static int check_attn(const mkv_t* h, const char* who, int layer, const float* q, int ntok, int maxtok, int n,
                      int start, const void* out) {
    if (!h || !q || !out) return fail(MKV_E_ARG, "%s: NULL argument", who);
    if (int rc = check_layer(h, layer)) return rc;
    if (ntok < 1 || ntok > maxtok) return fail(MKV_E_ARG, "%s: %d tokens outside [1, %d]", who, ntok, maxtok);
    if (n < 1 || start < 0 || start >= n) return fail(MKV_E_POS, "%s: n = %d, start = %d", who, n, start);
    if (n + ntok - 1 > h->len[layer])
        return fail(MKV_E_POS, "%s: reads positions up to %d, layer %d holds %d", who, n + ntok - 1, layer,
                    h->len[layer]);
    return MKV_OK;
}

static int decode_entry(const char* who, mkv_t* h, int layer, const float* q, int ntok, int n, int start, float scale,
                        void* out, bool h16, const float* gate) {
    if (int rc = check_attn(h, who, layer, q, ntok, 4, n, start, out)) return rc;
    if (h16 && !gate) return fail(MKV_E_ARG, "%s: the f16 output is the gated attention: gate_src is required", who);
    hipError_t e = decode_all(h, h->dws, layer, q, ntok, n, start, scale, out, h16, gate);
    return e == hipSuccess ? MKV_OK : hip_fail(e, who);
}

int mkv_decode(mkv_t* h, int layer, const float* q, int ntok, int n, int start, float scale, float* out,
               const float* gate) {
    return decode_entry("mkv_decode", h, layer, q, ntok, n, start, scale, out, false, gate);
}

int mkv_decode_g16(mkv_t* h, int layer, const float* q, int ntok, int n, int start, float scale, uint16_t* out16,
                   const float* gate) {
    return decode_entry("mkv_decode_g16", h, layer, q, ntok, n, start, scale, out16, true, gate);
}

static int append_decode(const char* who, mkv_t* h, const DecodeWs* ws, int layer, int n, int ntok, const float* kn,
                         const float* v, const float* tab, const float* q, int start, float scale, void* out,
                         bool h16, const float* gate) {
    if (ntok < 1 || ntok > 4) return fail(MKV_E_ARG, "%s: %d tokens outside [1, 4]", who, ntok);
    if (!h || !kn || !v || !tab) return fail(MKV_E_ARG, "%s: NULL argument", who);
    if (h16 && !gate) return fail(MKV_E_ARG, "%s: the f16 output is the gated attention: gate_src is required", who);
    if (int rc = check_layer(h, layer)) return rc;
    const int pos = n - 1;
    if (pos < 0 || pos + ntok > h->g.ctx)
        return fail(MKV_E_POS, "%s: positions [%d, %d) outside the context %d", who, pos, pos + ntok, h->g.ctx);
    if (pos > h->len[layer])
        return fail(MKV_E_POS, "%s: position %d leaves a hole after the written length %d", who, pos, h->len[layer]);
    const int old_len = h->len[layer];
    h->len[layer] = pos + ntok;
    if (int rc = check_attn(h, who, layer, q, ntok, 4, n, start, out)) {
        h->len[layer] = old_len;
        return rc;
    }
    if (!ws) ws = &h->dws;
    FusedAppend fa;
    fa.kn = kn;
    fa.v = v;
    fa.tab = tab;
    fa.pos = pos;
    fa.ntok = ntok;
    hipError_t e = decode_all(h, *ws, layer, q, ntok, n, start, scale, out, h16, gate, fa);
    if (e != hipSuccess) {
        h->len[layer] = old_len;
        return hip_fail(e, who);
    }
    return MKV_OK;
}

int mkv_append_decode(mkv_t* h, int layer, int n, int ntok, const float* kn, const float* v, const float* tab,
                      const float* q, int start, float scale, float* out, const float* gate) {
    return append_decode("mkv_append_decode", h, nullptr, layer, n, ntok, kn, v, tab, q, start, scale, out, false,
                         gate);
}

int mkv_append_decode_g16(mkv_t* h, int layer, int n, int ntok, const float* kn, const float* v, const float* tab,
                          const float* q, int start, float scale, uint16_t* out16, const float* gate) {
    return append_decode("mkv_append_decode_g16", h, nullptr, layer, n, ntok, kn, v, tab, q, start, scale, out16, true,
                         gate);
}

int mkv_append_decode_noalloc(mkv_t* h, int layer, int n, int ntok, const float* kn, const float* v,
                              const float* tab, const float* q, int start, float scale, float* out,
                              const float* gate) {
    if (!h) return fail(MKV_E_ARG, "mkv_append_decode_noalloc: NULL handle");
    float* sp = scratch_of(h->device);
    if (!sp) {  // not resolved by mkv_create: once more, if the handle's device is the current one
        int cur = -1;
        if (hipGetDevice(&cur) == hipSuccess && cur == h->device && resolve_scratch(cur) == hipSuccess)
            sp = scratch_of(cur);
    }
    if (!sp) return fail(MKV_E_HIP, "mkv_append_decode_noalloc: no scratch address for device %d", h->device);
    // the split plan of this call, checked against the scratch's capacity before anything is enqueued
    const int nch = h->g.fmt == MKV_F32 ? attn32_plan(ntok < 1 ? 1 : ntok, n, start).nch
                                        : decode_plan(n, ntok < 1 ? 1 : ntok, start).nch;
    if (nch > SCRATCH_CHUNKS)
        return fail(MKV_E_SIZE, "mkv_append_decode_noalloc: %d splits exceed the scratch's %d (%zu bytes)", nch,
                    SCRATCH_CHUNKS, SCRATCH_FLOATS * sizeof(float));
    const DecodeWs ws{sp, SCRATCH_CHUNKS};
    // no trace events on this path: taking them may create events and grows the pending list (host allocations)
    const bool tracing = h->tracing;
    h->tracing = false;
    const int rc = append_decode("mkv_append_decode_noalloc", h, &ws, layer, n, ntok, kn, v, tab, q, start, scale,
                                 out, false, gate);
    h->tracing = tracing;
    return rc;
}

size_t mkv_noalloc_scratch_bytes(void) { return SCRATCH_FLOATS * sizeof(float); }

int mkv_prefill(mkv_t* h, int layer, const float* q, int T, int n, int start, float scale, float* out,
                const float* gate) {
    if (int rc = check_attn(h, "mkv_prefill", layer, q, T, MKV_PREFILL_MAX, n, start, out)) return rc;
    hipError_t e = hipSuccess;
    int span = 0, nch = 0, rpk = T * GQA;  // the split-K plan the merge reads
    if (h->g.fmt == MKV_F16 && T <= SMALL_PREFILL_MAX) {
        // blocks under 64 tokens: f32-class, as the reference's attn_fd4 (engine.rs:1237-1241)
        const SmallPlan p = small_prefill_plan(T, n, start);
        if (small_prefill_ws_floats(T, p.d.nch) > h->pws_floats) return fail(MKV_E_ARG, "mkv_prefill: workspace");
        span = p.d.span;
        nch = p.d.nch;
        rpk = 32 * p.nzb;
        e = traced(h, MKV_SPAN_CORE, [&](const Launch& L) {
            return launch_small_prefill(h->g, h->base, layer, q, T, n, start, scale, p, h->pws, L);
        });
    } else {
        // f16: attn_fa_mx's arithmetic on 32-token work-groups; f32: 16-token work-groups, f32-class arithmetic
        const bool f16 = h->g.fmt == MKV_F16;
        const PrefillPlan p = f16 ? prefill_plan(T, n) : prefill32_plan(T, n);
        if (prefill_ws_floats(T, p.nch) > h->pws_floats) return fail(MKV_E_ARG, "mkv_prefill: workspace");
        span = p.span;
        nch = p.nch;
        e = traced(h, MKV_SPAN_CORE, [&](const Launch& L) {
            return f16 ? launch_prefill(h->g, h->base, layer, q, T, n, start, scale, p, h->pws, L)
                       : launch_prefill_f32(h->g, h->base, layer, q, T, n, start, scale, p, h->pws, L);
        });
    }
    if (e == hipSuccess)
        e = traced(h, MKV_SPAN_MERGE,
                   [&](const Launch& L) {
                       return launch_merge(h->pws, rpk, T, n, start, span, nch, gate, out, false, L);
                   });
    return e == hipSuccess ? MKV_OK : hip_fail(e, "mkv_prefill");
}

// Bytes of the [0, p) prefix of one plane of K (which = 0) or V (which = 1): whole layout units (K blocks of 32
// positions, V groups of 8 (f16) or 4 (f32) positions) of the store's own layout.
static size_t prefix_bytes(const mkv_t* h, int which, int p) {
    const int unit = plane_unit(h->g.fmt, which);
    return (size_t)((p + unit - 1) / unit) * unit * HD * h->g.bpe();
}

size_t mkv_snapshot_bytes(const mkv_t* h, int p) {
    if (!h || p < 0 || p > h->g.ctx) return 0;
    return (size_t)h->g.layers * KVH * (prefix_bytes(h, 0, p) + prefix_bytes(h, 1, p));
}

static int snap_copy(mkv_t* h, int p, void* host, const void* chost, size_t bytes, bool save) {
    const char* who = save ? "mkv_snapshot" : "mkv_restore";
    if (!h || (!host && !chost)) return fail(MKV_E_ARG, "%s: NULL argument", who);
    if (p < 0 || p > h->g.ctx) return fail(MKV_E_POS, "%s: p = %d outside [0, %d]", who, p, h->g.ctx);
    if (save)
        for (int l = 0; l < h->g.layers; l++)
            if (p > h->len[l]) return fail(MKV_E_POS, "%s: p = %d past the written length %d of layer %d", who, p,
                                           h->len[l], l);
    if (bytes != mkv_snapshot_bytes(h, p))
        return fail(MKV_E_SIZE, "%s: %zu bytes given, %zu needed for %d positions", who, bytes,
                    mkv_snapshot_bytes(h, p), p);
    {
        // the copies are asynchronous on the stream: only pinned host memory may take them (pageable memory would
        // make the runtime stage and block, and a restore would read the caller's buffer after this call returns)
        hipPointerAttribute_t a{};
        const hipError_t pe = hipPointerGetAttributes(&a, save ? host : chost);
        if (pe != hipSuccess) (void)hipGetLastError();  // an unknown (pageable) pointer: clear the error it recorded
        if (pe != hipSuccess || a.type != hipMemoryTypeHost)
            return fail(MKV_E_ARG, "%s: the host buffer is not pinned host memory (hipHostMalloc)", who);
    }
    if (p == 0) {
        if (!save) h->len.assign(h->g.layers, 0);
        return MKV_OK;
    }
    // image order: for each layer, K planes (kvh 0, 1) then V planes (kvh 0, 1); each plane's prefix is one row of a
    // 2D copy with the plane size as device pitch
    const size_t kb = prefix_bytes(h, 0, p), vb = prefix_bytes(h, 1, p);
    const size_t pb = h->g.plane_bytes();
    char* dev = (char*)h->base;
    char* hb = (char*)(save ? host : const_cast<void*>(chost));
    hipError_t e = hipSuccess;
    if (kb == vb) {
        int rows = h->g.layers * 2 * KVH;
        e = save ? hipMemcpy2DAsync(hb, kb, dev, pb, kb, rows, hipMemcpyDeviceToHost, h->stream)
                 : hipMemcpy2DAsync(dev, pb, hb, kb, kb, rows, hipMemcpyHostToDevice, h->stream);
    } else {
        size_t off = 0;
        for (int l = 0; l < h->g.layers && e == hipSuccess; l++) {
            for (int which = 0; which < 2 && e == hipSuccess; which++) {
                size_t w = which == 0 ? kb : vb;
                char* d = dev + h->g.plane(l, which, 0) * pb;
                e = save ? hipMemcpy2DAsync(hb + off, w, d, pb, w, KVH, hipMemcpyDeviceToHost, h->stream)
                         : hipMemcpy2DAsync(d, pb, hb + off, w, w, KVH, hipMemcpyHostToDevice, h->stream);
                off += w * KVH;
            }
        }
    }
    if (e == hipSuccess && save) e = hipStreamSynchronize(h->stream);
    if (e != hipSuccess) return hip_fail(e, who);
    if (!save) h->len.assign(h->g.layers, p);
    return MKV_OK;
}

int mkv_snapshot(mkv_t* h, int p, void* host, size_t bytes) { return snap_copy(h, p, host, nullptr, bytes, true); }

int mkv_restore(mkv_t* h, int p, const void* host, size_t bytes) {
    return snap_copy(h, p, nullptr, host, bytes, false);
}

int mkv_read_rows(mkv_t* h, int layer, int which, int p0, int p1, void* dst) {
    if (!h || (!dst && p1 != p0)) return fail(MKV_E_ARG, "mkv_read_rows: NULL argument");
    if (int rc = check_layer(h, layer)) return rc;
    if (which != MKV_K && which != MKV_V) return fail(MKV_E_ARG, "mkv_read_rows: which = %d", which);
    if (p0 < 0 || p1 < p0 || p1 > h->g.ctx) return fail(MKV_E_POS, "mkv_read_rows: [%d, %d)", p0, p1);
    hipError_t e = launch_read_rows(h->g, h->base, layer, which, p0, p1, dst, Launch{h->stream});
    return e == hipSuccess ? MKV_OK : hip_fail(e, "mkv_read_rows");
}

int mkv_write_rows(mkv_t* h, int layer, int which, int p0, int p1, const void* src) {
    if (!h || (!src && p1 != p0)) return fail(MKV_E_ARG, "mkv_write_rows: NULL argument");
    if (int rc = check_layer(h, layer)) return rc;
    if (which != MKV_K && which != MKV_V) return fail(MKV_E_ARG, "mkv_write_rows: which = %d", which);
    if (p0 < 0 || p1 < p0 || p1 > h->g.ctx) return fail(MKV_E_POS, "mkv_write_rows: [%d, %d)", p0, p1);
    if (p0 > h->len[layer])
        return fail(MKV_E_POS, "mkv_write_rows: position %d leaves a hole after the written length %d", p0,
                    h->len[layer]);
    hipError_t e = launch_write_rows(h->g, h->base, layer, which, p0, p1, src, Launch{h->stream});
    if (e != hipSuccess) return hip_fail(e, "mkv_write_rows");
    if (p1 > h->len[layer]) h->len[layer] = p1;
    return MKV_OK;
}

int mkv_trace(mkv_t* h, int enable) {
    if (!h) return fail(MKV_E_ARG, "mkv_trace: NULL handle");
    if (enable) {
        hipError_t e = hipStreamSynchronize(h->stream);
        if (e != hipSuccess) return hip_fail(e, "mkv_trace");
        for (auto& s : h->pending) {
            h->pool.push_back(s.a);
            h->pool.push_back(s.b);
        }
        h->pending.clear();
        for (int i = 0; i < MKV_SPANS; i++) {
            h->ms[i] = 0;
            h->count[i] = 0;
        }
        // events for the traced launches, created (and recorded once) here, so that no event is created while the
        // traced launches are being enqueued
        while (h->pool.size() < TRACE_RESERVE) {
            hipEvent_t ev = nullptr;
            e = hipEventCreate(&ev);
            if (e == hipSuccess) e = hipEventRecord(ev, h->stream);
            if (e != hipSuccess) {
                if (ev) (void)hipEventDestroy(ev);
                return hip_fail(e, "mkv_trace: events");
            }
            h->pool.push_back(ev);
        }
        e = hipStreamSynchronize(h->stream);
        if (e != hipSuccess) return hip_fail(e, "mkv_trace");
    }
    h->tracing = enable != 0;
    return MKV_OK;
}

int mkv_trace_read(mkv_t* h, double* ms, long* count) {
    if (!h || !ms || !count) return fail(MKV_E_ARG, "mkv_trace_read: NULL argument");
    hipError_t e = hipStreamSynchronize(h->stream);
    if (e != hipSuccess) return hip_fail(e, "mkv_trace_read");
    for (auto& s : h->pending) {
        float t = 0.f;
        e = hipEventElapsedTime(&t, s.a, s.b);
        if (e != hipSuccess) return hip_fail(e, "mkv_trace_read: elapsed time");
        h->ms[s.kind] += t;
        h->count[s.kind] += 1;
        h->pool.push_back(s.a);
        h->pool.push_back(s.b);
    }
    h->pending.clear();
    for (int i = 0; i < MKV_SPANS; i++) {
        ms[i] = h->ms[i];
        count[i] = h->count[i];
    }
    return MKV_OK;
}

int mkv_rope_table(int pos, float* tab) {
    if (!tab) return fail(MKV_E_ARG, "mkv_rope_table: NULL argument");
    // engine.rs:108-114: f32 throughout; Rust's f32 powf / cos / sin are the platform libm's powf / cosf / sinf
    float scale = powf(1e7f, -2.0f / 64.0f);
    float th = (float)pos;
    for (int i = 0; i < 32; i++) {
        tab[i] = cosf(th);
        tab[32 + i] = sinf(th);
        th = th * scale;
    }
    return MKV_OK;
}

int mkv_rope_table_dev(mkv_t* h, int pos, const float** tab) {
    if (!h || !tab) return fail(MKV_E_ARG, "mkv_rope_table_dev: NULL argument");
    if (pos < 0 || pos >= h->g.ctx) return fail(MKV_E_POS, "mkv_rope_table_dev: position %d outside [0, %d)", pos,
                                              h->g.ctx);
    if (!h->rope_dev) {
        std::vector<float> t((size_t)h->g.ctx * 64);
        for (int p = 0; p < h->g.ctx; p++) mkv_rope_table(p, t.data() + (size_t)p * 64);
        float* d = nullptr;
        if (hipMalloc(&d, t.size() * sizeof(float)) != hipSuccess)
            return fail(MKV_E_NOMEM, "mkv_rope_table_dev: %zu bytes", t.size() * sizeof(float));
        hipError_t e = hipMemcpy(d, t.data(), t.size() * sizeof(float), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(d);
            return hip_fail(e, "mkv_rope_table_dev");
        }
        h->rope_dev = d;
    }
    *tab = h->rope_dev + (size_t)pos * 64;
    return MKV_OK;
}

int mkv_qk_norm_rope(mkv_t* h, int pos, int ntok, const float* qf, const float* kb, const float* q_norm_w,
                     const float* k_norm_w, float eps, float* q_out, float* kn_out) {
    if (!h || !qf || !kb || !q_norm_w || !k_norm_w || !q_out || !kn_out)
        return fail(MKV_E_ARG, "mkv_qk_norm_rope: NULL argument");
    if (ntok < 1 || ntok > MKV_PREFILL_MAX) return fail(MKV_E_ARG, "mkv_qk_norm_rope: ntok %d outside [1, %d]", ntok,
                                                       MKV_PREFILL_MAX);
    if (pos < 0 || pos + ntok > h->g.ctx)
        return fail(MKV_E_POS, "mkv_qk_norm_rope: positions [%d, %d) outside the context %d", pos, pos + ntok,
                    h->g.ctx);
    const float* tab = nullptr;
    if (int rc = mkv_rope_table_dev(h, pos, &tab)) return rc;
    hipError_t e = launch_qk_produce(ntok, qf, kb, q_norm_w, k_norm_w, eps, tab, q_out, kn_out, Launch{h->stream});
    return e == hipSuccess ? MKV_OK : hip_fail(e, "mkv_qk_norm_rope");
}

}  // extern "C"
