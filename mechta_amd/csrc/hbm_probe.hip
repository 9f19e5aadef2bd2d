// hbm_probe.hip -- measurement aid for bench.py, not part of the KV-cache ABI: the time one launch takes to read a
// buffer of a given size from HBM with nothing else to do, so that the decode kernel's rate can be read against what
// a plain streaming read of the same bytes reaches on this GPU.
//
// Each of `wgs` work-groups (512 threads) reads 64 KB stages dealt round robin (stage u to work-group u % wgs, as the
// decode deals its stages) with 16-byte non-temporal buffer loads, two stages in flight, and folds the words with xor
// (written out only on an impossible value, so the loads stay live). Durations come from the dispatch packet's
// timestamps (hipExtLaunchKernel events), as the library's kernel trace takes them.
#include <hip/hip_runtime.h>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int STAGE = 65536;

__device__ inline __amdgpu_buffer_rsrc_t rsrc(const char* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

__global__ void __launch_bounds__(512) probe_read(const char* __restrict__ p, unsigned nst, unsigned* __restrict__ out) {
    const unsigned nwg = gridDim.x, c = blockIdx.x, t = threadIdx.x;
    const unsigned per = (nst + nwg - 1) / nwg;
    u32x4 acc = {0, 0, 0, 0};
    u32x4 b0[8], b1[8];
    auto load = [&](unsigned j, u32x4* b) {  // stage j of this work-group; past the end: out of range, no bytes
        const unsigned u = j * nwg + c;
        const __amdgpu_buffer_rsrc_t r = rsrc(p + (size_t)(u < nst ? u : 0) * STAGE, u < nst ? STAGE : 0);
#pragma unroll
        for (int i = 0; i < 8; i++) b[i] = __builtin_amdgcn_raw_buffer_load_b128(r, (i * 512 + t) * 16, 0, 2);
    };
    load(0, b0);
    load(1, b1);
    for (unsigned j = 0; j < per; j += 2) {
#pragma unroll
        for (int i = 0; i < 8; i++) acc ^= b0[i];
        load(j + 2, b0);
#pragma unroll
        for (int i = 0; i < 8; i++) acc ^= b1[i];
        load(j + 3, b1);
    }
    if (acc.x == 0x9E3779B9u && acc.y == 0x7F4A7C15u) out[c] = acc.z;
}

}  // namespace

// Reads each of the nbuf device buffers (bytes each, a multiple of 64 KB) in turn, reps launches in all, on the null
// stream; *mean_us and *best_us receive the launch durations. Returns 0, or a HIP error code.
extern "C" int mkv_probe_read(const void* const* bufs, int nbuf, size_t bytes, int wgs, int reps, float* mean_us,
                              float* best_us) {
    if (nbuf < 1 || reps < 1 || wgs < 1 || bytes % STAGE || bytes / STAGE > 0xFFFFFFFFull) return (int)hipErrorInvalidValue;
    unsigned* out = nullptr;
    hipError_t e = hipMalloc(&out, (size_t)wgs * sizeof(unsigned));
    if (e != hipSuccess) return (int)e;
    hipEvent_t a, b;
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    double sum = 0.0;
    float best = 1e30f;
    for (int i = 0; i < reps && e == hipSuccess; i++) {
        const char* p = (const char*)bufs[i % nbuf];
        unsigned nst = (unsigned)(bytes / STAGE);
        void* args[] = {(void*)&p, (void*)&nst, (void*)&out};
        e = hipExtLaunchKernel((const void*)probe_read, dim3(wgs), dim3(512), args, 0, nullptr, a, b, 0);
        if (e == hipSuccess) e = hipEventSynchronize(b);
        float ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
        sum += ms * 1e3;
        best = ms * 1e3f < best ? ms * 1e3f : best;
    }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    (void)hipFree(out);
    *mean_us = (float)(sum / reps);
    *best_us = best;
    return (int)e;
}
