// mkv_store.h -- the store object shared by the C ABI's source files (kv_store.cpp, kv_root.cpp).
#pragma once
#include <hip/hip_runtime.h>

#include <thread>
#include <vector>

#include "../../include/mechta_kv.h"
#include "mkv_internal.h"

// One KV store: geometry, the one HBM allocation of every plane, the stream, per-layer lengths, the split-K
// workspaces, the trace spans.
struct mkv_store {
    mkv::Geom g;
    void* base = nullptr;           // layers x {K, V} x 2 planes
    hipStream_t stream = nullptr;
    int device = 0;                 // the device current at mkv_create
    std::vector<int> len;           // written positions per layer
    mkv::DecodeWs dws{nullptr, 0};
    float* pws = nullptr;           // prefill partials
    size_t pws_floats = 0;
    // tracing: events bracketing each kernel launch while on
    bool tracing = false;
    struct Span {
        int kind;
        hipEvent_t a, b;
    };
    std::vector<Span> pending;
    std::vector<hipEvent_t> pool;
    double ms[MKV_SPANS] = {0, 0, 0};
    long count[MKV_SPANS] = {0, 0, 0};
    // RoPE table rows of every position [0, ctx) on the device (built on first use from mkv_rope_table)
    float* rope_dev = nullptr;
    // root file written in the background (mkv_root_save with background != 0) from pinned host memory
    std::thread root_thread;
    int root_rc = 0;
    char root_err[512] = "";
    void* root_host = nullptr;      // pinned host buffer of root saves and loads, reused (grown when too small)
    size_t root_cap = 0;
};


namespace mkv {
extern thread_local char g_err[512];
int fail(int code, const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);
void root_join(mkv_store* h);  // waits for a background root write
void root_free(mkv_store* h);  // joins, then frees the pinned root buffer
}  // namespace mkv
