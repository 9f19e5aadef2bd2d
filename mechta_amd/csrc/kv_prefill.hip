// kv_prefill.hip -- causal prefill flash attention (placeholder: the store falls back to the decode kernel).
#include "mkv_internal.h"

namespace mkv {

size_t prefill_ws_floats(int ctx) { (void)ctx; return 0; }

hipError_t launch_prefill(const Geom& g, const void* base, int layer, const float* q, int T, int n, int start,
                          float scale, float* ws, size_t ws_floats, const Launch& L) {
    (void)g; (void)base; (void)layer; (void)q; (void)T; (void)n; (void)start; (void)scale; (void)ws; (void)ws_floats;
    (void)L;
    return hipErrorNotSupported;
}

hipError_t launch_prefill_merge(int T, int n, int start, float* ws, const float* gate, float* out, const Launch& L) {
    (void)T; (void)n; (void)start; (void)ws; (void)gate; (void)out; (void)L;
    return hipErrorNotSupported;
}

}  // namespace mkv
