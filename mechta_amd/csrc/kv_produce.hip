// kv_produce.hip -- the q/k producer in front of the append: per-head RMSNorm of q and k and the RoPE of q, one
// kernel for what the reference dispatches as rmsnorm (q), rmsnorm (k) and rope2 (q) (quad.rs:113-115,
// engine.rs:1210-1212; kernels ops.wgsl:27-57 and :275-286). The k rows leave normed and unrotated: their rotation
// and f16 rounding are the append's (mkv_append / mkv_append_decode), as kv_rope2 does them in the reference.
//
// One wave per 256-value row (16 q rows and 2 k rows per token). The row's sum of squares follows the reference's
// 256-thread shared-memory tree exactly (partial[t] += partial[t + m], m = 128 .. 1): lane l holds x[l], x[l+64],
// x[l+128], x[l+192]; m = 128 and 64 are additions inside the lane, m = 32 .. 1 lane shifts. With the square root
// and division correctly rounded and no contraction (the file is also built with -ffp-contract=off) the result is
// bit-identical to that reduction.
#include "mkv_device.h"

namespace mkv {
namespace {

__global__ void __launch_bounds__(64) qk_produce(const float* __restrict__ qf, const float* __restrict__ kb,
                                                 const float* __restrict__ q_w, const float* __restrict__ k_w,
                                                 float eps, const float* __restrict__ tab, float* __restrict__ q_out,
                                                 float* __restrict__ kn_out) {
#pragma clang fp contract(off)
    const int t = blockIdx.x / (QH + KVH), r = blockIdx.x % (QH + KVH), l = threadIdx.x;
    const bool isq = r < QH;
    const float* x = isq ? qf + ((size_t)t * QH + r) * 512 : kb + ((size_t)t * KVH + (r - QH)) * HD;
    const float* w = isq ? q_w : k_w;
    float v[4], s[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        v[j] = x[l + 64 * j];
        s[j] = v[j] * v[j];
    }
    // m = 128: partial[t] = partial[t] + partial[t + 128] for t = l, l + 64; m = 64: partial[l] += partial[l + 64]
    float p = (s[0] + s[2]) + (s[1] + s[3]);
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) p = p + __shfl_down(p, m);  // lanes < m hold partial[l]
    const float sum = __shfl(p, 0);  // partial[0]
    // sqrtf: correctly rounded (v_sqrt_f32 then the neighbours checked by FMA residuals); __fsqrt_rn is not
    const float scale = __fdiv_rn(1.0f, sqrtf(sum * (1.0f / 256.0f) + eps));  // sum / 256 is exact
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; j++) y[j] = (v[j] * scale) * w[l + 64 * j];
    if (!isq) {
        float* o = kn_out + ((size_t)t * KVH + (r - QH)) * HD;
#pragma unroll
        for (int j = 0; j < 4; j++) o[l + 64 * j] = y[j];
        return;
    }
    // rope2 on dims 0..63 (pairs i, i + 32 of y[0]); lanes 32..63 hold the second halves
    const float* tb = tab + (size_t)t * 64;
    const float other = __shfl_xor(y[0], 32);
    const int i = l & 31;
    const float c = tb[i], sn = tb[32 + i];
    float o0;
    if (l < 32) o0 = y[0] * c - other * sn;  // x1 c - x2 s
    else o0 = other * sn + y[0] * c;         // x1 s + x2 c
    float* o = q_out + ((size_t)t * QH + r) * HD;
    o[l] = o0;
#pragma unroll
    for (int j = 1; j < 4; j++) o[l + 64 * j] = y[j];
}

}  // namespace

hipError_t launch_qk_produce(int ntok, const float* qf, const float* kb, const float* q_w, const float* k_w,
                             float eps, const float* tab, float* q_out, float* kn_out, const Launch& L) {
    return launch(qk_produce, dim3(ntok * (QH + KVH)), dim3(64), L, qf, kb, q_w, k_w, eps, tab, q_out, kn_out);
}

}  // namespace mkv
