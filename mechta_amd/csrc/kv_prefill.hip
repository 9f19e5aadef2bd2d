// kv_prefill.hip -- causal prefill flash attention (placeholder: the store falls back to the decode kernel).
#include "mkv_internal.h"

namespace mkv {

size_t prefill_ws_floats(int ctx) { (void)ctx; return 0; }

hipError_t launch_prefill(const Geom& g, const void* base, int layer, const float* q, int T, int n, int start,
                          float scale, float* out, const float* gate, float* ws, size_t ws_floats, hipStream_t s) {
    (void)g; (void)base; (void)layer; (void)q; (void)T; (void)n; (void)start; (void)scale; (void)out; (void)gate;
    (void)ws; (void)ws_floats; (void)s;
    return hipErrorNotSupported;
}

}  // namespace mkv
