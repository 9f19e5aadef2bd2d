// hbm_probe.hip -- measurement aid for bench.py, not part of the KV-cache ABI: the time one launch takes to read a
// buffer of a given size from HBM with nothing else to do, so that the decode kernel's rate can be read against what
// a plain streaming read of the same bytes reaches on this GPU, and how that rate depends on the launch shape; and
// (at the end of the file) the dense f16 rate the matrix units sustain, the same for the prefill kernels.
//
// Each of `wgs` work-groups (`threads` threads) reads stages of threads x 128 bytes (8 x 16-byte loads per thread),
// dealt round robin (stage u to work-group u % wgs, as the decode deals its stages; optionally skewed, half the
// work-groups ending a few stages before the other half) or as one contiguous range per work-group, with DEPTH stages in flight per work-group, 16-byte buffer loads (non-temporal or default policy), and
// folds the words with xor (written out only on an impossible value, so the loads stay live). Optionally every
// work-group writes `tail` bytes at its end (as the decode writes its split-K partials), 16-byte stores with a chosen
// cache policy. Durations come from the
// dispatch packet's timestamps (hipExtLaunchKernel events), as the library's kernel trace takes them; `wall` is the
// time per launch of `reps` launches back to back on one stream (what a step of back-to-back launches costs).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int LOADS = 8;  // 16-byte loads per thread and stage

__device__ inline __amdgpu_buffer_rsrc_t rsrc(const char* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

template <int DEPTH, int POL, bool RR, int MAXT>  // MAXT: the launch's threads at most (the register budget follows)
__global__ void __launch_bounds__(MAXT) probe_read(const char* __restrict__ p, unsigned nst, unsigned* __restrict__ out,
                                                   unsigned tail_words, int tail_pol, unsigned skew) {
    const unsigned nwg = gridDim.x, c = blockIdx.x, t = threadIdx.x, nt = blockDim.x;
    const unsigned stage = nt * LOADS * 16;
    const unsigned per0 = (nst + nwg - 1) / nwg;
    // skew (round robin, even nwg): the first per0 - skew rounds go to every work-group, the last 2 skew rounds' stages
    // to the odd work-groups only, so half the grid ends skew stages early and the other half skew stages late
    const unsigned base = skew ? (per0 - skew) * nwg : 0;
    const unsigned per = !skew ? per0 : (c & 1) ? per0 + skew : per0 - skew;
    u32x4 acc = {0, 0, 0, 0};
    u32x4 b[DEPTH][LOADS];
    auto load = [&](unsigned j, u32x4* bb) {  // stage j of this work-group; past the end: out of range, no bytes
        const unsigned u = !RR ? c * per + j : j < per0 - skew || !skew ? j * nwg + c
                                                                         : base + (j - (per0 - skew)) * (nwg / 2) + c / 2;
        const bool ok = j < per && u < nst;
        const __amdgpu_buffer_rsrc_t r = rsrc(p + (size_t)(ok ? u : 0) * stage, ok ? stage : 0);
#pragma unroll
        for (int i = 0; i < LOADS; i++) bb[i] = __builtin_amdgcn_raw_buffer_load_b128(r, (i * nt + t) * 16, 0, POL);
    };
#pragma unroll
    for (int d = 0; d < DEPTH; d++) load(d, b[d]);
    for (unsigned j = 0; j < per; j += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; d++) {
#pragma unroll
            for (int i = 0; i < LOADS; i++) acc ^= b[d][i];
            load(j + d + DEPTH, b[d]);
        }
    }
    if (acc.x == 0x9E3779B9u && acc.y == 0x7F4A7C15u) out[c] = acc.z;
    // tail write, 16 bytes per store: policy 0 plain (write-back L2), 1 sc1 (device scope), 2 nt, 3 sc0 sc1
    const __amdgpu_buffer_rsrc_t tr = rsrc((const char*)(out + nwg + (size_t)c * tail_words), tail_words * 4);
    for (unsigned i = t; i < tail_words / 4; i += nt) {
        const u32x4 v = {acc.w + i, acc.x, acc.y, acc.z};
        if (tail_pol == 1) __builtin_amdgcn_raw_buffer_store_b128(v, tr, i * 16, 0, 16);
        else if (tail_pol == 2) __builtin_amdgcn_raw_buffer_store_b128(v, tr, i * 16, 0, 2);
        else if (tail_pol == 3) __builtin_amdgcn_raw_buffer_store_b128(v, tr, i * 16, 0, 17);
        else __builtin_amdgcn_raw_buffer_store_b128(v, tr, i * 16, 0, 0);
    }
}

// The read of probe_read<2, nt, round robin> followed by the tail a split-K decode would need to merge its own
// partials in the same launch: every work-group writes a 33,280-byte partial (32 rows x 260 floats), the work-groups
// of each half of the grid (the work-groups of one kv head) meet at a barrier, and each then reads its share of the
// half's partials as a merge would (a 64-dim slice of one row from every partial, 16 chunk lanes x 16 dim lanes in one
// round trip) and writes 256 bytes. Every wait is bounded (a work-group that gives up marks itself in out[]). Modes:
//   1  the partial stores only (plain stores), no barrier or merge
//   2  plain partial stores, __threadfence() in every wave (agent-scope release/acquire: L2 write-back and
//      invalidate), merge reads without any counter (timing only)
//   3  as 2, plus one relaxed arrival atomic per work-group, no wait
//   4, 5  as 2, then the barrier: one arrival counter per half, the last arrival advances a generation word that the
//      others poll (s_sleep 1 / 20 between polls)
//   6, 7  device-coherent partials instead (16-byte stores with scope bit sc1, written through the XCD's L2, so no
//      fence is needed: each wave waits for its stores), relaxed counter and generation as 4, merge reads with sc1
//   8  as 6 with the arrival atomic only, no wait
//   9  as 6 with 8 sub-counters (work-groups gi % 8) whose last arrivals count at the top counter
//   10 as 6 with one flag per work-group set to the launch's epoch, polled by wave 0 (one load per work-group)
constexpr int FUSED_PART = 32 * 260;  // floats per partial
__global__ void __launch_bounds__(512) probe_fused(const char* __restrict__ p, unsigned nst, unsigned* __restrict__ out,
                                                   float* __restrict__ part, unsigned* __restrict__ sync,
                                                   int mode, unsigned epoch) {
    const unsigned nwg = gridDim.x, c = blockIdx.x, t = threadIdx.x, nt = blockDim.x;
    const unsigned stage = nt * LOADS * 16;
    const unsigned per = (nst + nwg - 1) / nwg;
    const unsigned grp = c & 1, ng = nwg / 2, gi = c >> 1;
    u32x4 acc = {0, 0, 0, 0};
    u32x4 b[2][LOADS];
    auto load = [&](unsigned j, u32x4* bb) {
        const unsigned u = j * nwg + c;
        const bool ok = j < per && u < nst;
        const __amdgpu_buffer_rsrc_t r = rsrc(p + (size_t)(ok ? u : 0) * stage, ok ? stage : 0);
#pragma unroll
        for (int i = 0; i < LOADS; i++) bb[i] = __builtin_amdgcn_raw_buffer_load_b128(r, (i * nt + t) * 16, 0, 2);
    };
    load(0, b[0]);
    load(1, b[1]);
    for (unsigned j = 0; j < per; j += 2) {
#pragma unroll
        for (int d = 0; d < 2; d++) {
#pragma unroll
            for (int i = 0; i < LOADS; i++) acc ^= b[d][i];
            load(j + d + 2, b[d]);
        }
    }
    float* mine = part + ((size_t)grp * ng + gi) * FUSED_PART;
    __shared__ int ok;
    if (mode >= 6) {
        // device-coherent partials: stores with scope bit sc1 go through the XCD's L2, so no L2 write-back (and no
        // invalidate on the reading side, whose loads carry sc1 too) is needed; the counters are relaxed atomics
        const __amdgpu_buffer_rsrc_t pr = rsrc((const char*)mine, FUSED_PART * 4);
        for (unsigned i = t; i < FUSED_PART / 4; i += nt)
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{acc.x + i, acc.y, acc.z, acc.w}, pr, i * 16, 0, 16);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (mode == 8 && t == 0) {  // arrivals only, no wait
            __hip_atomic_fetch_add(sync + 2 * grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = 1;
        }
        if (mode == 10 && t < 64) {  // one flag per work-group, set to this launch's epoch; wave 0 polls all of them
            if (t == 0) __hip_atomic_store(sync + 4096 + (grp * ng + gi) * 32, epoch, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
            int done = 0;
            for (int it = 0; it < (1 << 20); it++) {
                bool mine_ok = true;
                for (unsigned j = t; j < ng; j += 64)
                    mine_ok &= __hip_atomic_load(sync + 4096 + (grp * ng + j) * 32, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT) == epoch;
                if (__all(mine_ok)) {
                    done = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            if (t == 0) ok = done;
        }
        if ((mode == 6 || mode == 7 || mode == 9) && t == 0) {
            unsigned* cnt = sync + 1024 * grp;
            unsigned* gen = cnt + 1;
            const unsigned g0 = __hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            bool last;
            if (mode == 9) {  // 8 sub-counters (work-groups gi % 8), the last of each arrives at the top counter
                const unsigned sub = gi % 8, nsub = (ng - sub + 7) / 8;
                unsigned* sc = cnt + 64 * (sub + 1);
                last = __hip_atomic_fetch_add(sc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nsub - 1;
                if (last) {
                    __hip_atomic_store(sc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                           (ng < 8 ? ng : 8) - 1;
                }
            } else {
                last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ng - 1;
            }
            int done = 0;
            if (last) {
                __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_fetch_add(gen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                done = 1;
            } else {
                for (int it = 0; it < (1 << 20); it++) {
                    if (__hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != g0) {
                        done = 1;
                        break;
                    }
                    if (mode == 7) __builtin_amdgcn_s_sleep(8);
                    else __builtin_amdgcn_s_sleep(1);
                }
            }
            ok = done;
        }
        __syncthreads();
        const unsigned half = t >> 8, tt = t & 255, task = gi + half * ng;
        if (task < 128 && ok) {
            const unsigned row = task % 32, d0 = (task / 32) * 64 + (tt & 15) * 4, cl = tt >> 4;
            const __amdgpu_buffer_rsrc_t br =
                rsrc((const char*)(part + (size_t)grp * ng * FUSED_PART), ng * FUSED_PART * 4);
            u32x4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const unsigned ch = cl + 16 * j;
                v[j] = __builtin_amdgcn_raw_buffer_load_b128(
                    br, ch < ng ? (ch * FUSED_PART + row * 260 + 4 + d0) * 4 : 0x7FFFFFF0u, 0, 16);
            }
            u32x4 s = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 8; j++) s ^= v[j];
            ((u32x4*)(out + nwg))[(size_t)(grp * 128 + task) * 16 + (tt & 15)] = s;
        }
        if (!ok && t == 0) out[c] = 0xDEAD;
        return;
    }
    for (unsigned i = t; i < FUSED_PART; i += nt) mine[i] = (float)(acc.x & 0xFF) + (float)i;
    // barrier of the half: stores visible at agent scope, then one arrival per work-group
    if (mode == 1) return;
    __threadfence();
    __syncthreads();
    if (mode == 2) ok = 1;
    if (t == 0 && mode == 3) {
        __hip_atomic_fetch_add(sync + 2 * grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = 1;
    }
    if (t == 0 && mode >= 4) {
        unsigned* cnt = sync + 2 * grp;
        unsigned* gen = cnt + 1;
        const unsigned g0 = __hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        int done = 0;
        if (old == ng - 1) {
            __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(gen, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            done = 1;
        } else {
            for (int it = 0; it < (1 << 20); it++) {
                if (__hip_atomic_load(gen, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) != g0) {
                    done = 1;
                    break;
                }
                if (mode == 4) __builtin_amdgcn_s_sleep(1);
                else __builtin_amdgcn_s_sleep(20);
            }
        }
        ok = done;
    }
    __syncthreads();
    // merge share: work-group gi of the half takes row gi % 32, dims 64 (gi / 32 % 4) .. + 63 (two tasks per
    // work-group: threads 0..255 and 256..511)
    const unsigned half = t >> 8, tt = t & 255, task = gi + half * ng;
    if (task < 128 && ok) {
        const unsigned row = task % 32, d0 = (task / 32) * 64 + (tt & 15) * 4, cl = tt >> 4;
        const float* base = part + (size_t)grp * ng * FUSED_PART;
        float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const unsigned ch = cl + 16 * j;
            v[j] = ch < ng ? *(const float4*)(base + (size_t)ch * FUSED_PART + row * 260 + 4 + d0)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            s.x += v[j].x;
            s.y += v[j].y;
            s.z += v[j].z;
            s.w += v[j].w;
        }
        if (s.x == 1.2345f) out[c] = 1;
        ((float4*)(out + nwg))[(size_t)(grp * 128 + task) * 16 + (tt & 15)] = s;
    }
    if (!ok && t == 0) out[c] = 0xDEAD;
}

int g_tail_pol = 0;
unsigned g_skew = 0;

template <int DEPTH, int POL, bool RR>
hipError_t launch_one(const char* p, unsigned nst, unsigned* out, unsigned tail_words, int wgs, int threads,
                      hipEvent_t a, hipEvent_t b) {
    void* args[] = {(void*)&p, (void*)&nst, (void*)&out, (void*)&tail_words, (void*)&g_tail_pol, (void*)&g_skew};
    // the kernel built for the smallest thread bound that holds the launch: at 1024 threads a lane has 128 registers,
    // which 3 or 4 stages in flight (96 or 128 of them for the loads alone) would spill
    const void* k = threads <= 256   ? (const void*)probe_read<DEPTH, POL, RR, 256>
                    : threads <= 512 ? (const void*)probe_read<DEPTH, POL, RR, 512>
                                     : (const void*)probe_read<DEPTH, POL, RR, 1024>;
    return hipExtLaunchKernel(k, dim3(wgs), dim3(threads), args, 0, nullptr, a, b, 0);
}

template <int POL, bool RR>
hipError_t launch_depth(int depth, const char* p, unsigned nst, unsigned* out, unsigned tail_words, int wgs,
                        int threads, hipEvent_t a, hipEvent_t b) {
    switch (depth) {
        case 1: return launch_one<1, POL, RR>(p, nst, out, tail_words, wgs, threads, a, b);
        case 2: return launch_one<2, POL, RR>(p, nst, out, tail_words, wgs, threads, a, b);
        case 3: return launch_one<3, POL, RR>(p, nst, out, tail_words, wgs, threads, a, b);
        case 4: return launch_one<4, POL, RR>(p, nst, out, tail_words, wgs, threads, a, b);
        default: return hipErrorInvalidValue;
    }
}

int g_fused_mode = 4;
unsigned g_epoch = 0;
float* g_fused_part = nullptr;
unsigned* g_fused_sync = nullptr;

hipError_t launch_any(int depth, int nt_policy, int rr, const char* p, unsigned nst, unsigned* out,
                      unsigned tail_words, int wgs, int threads, hipEvent_t a, hipEvent_t b) {
    if (depth <= 0) {  // fused tail (probe_fused)
        g_epoch++;
        void* args[] = {(void*)&p, (void*)&nst, (void*)&out, (void*)&g_fused_part, (void*)&g_fused_sync,
                        (void*)&g_fused_mode, (void*)&g_epoch};
        return hipExtLaunchKernel((const void*)probe_fused, dim3(wgs), dim3(threads), args, 0, nullptr, a, b, 0);
    }
    if (nt_policy && rr) return launch_depth<2, true>(depth, p, nst, out, tail_words, wgs, threads, a, b);
    if (nt_policy) return launch_depth<2, false>(depth, p, nst, out, tail_words, wgs, threads, a, b);
    if (rr) return launch_depth<0, true>(depth, p, nst, out, tail_words, wgs, threads, a, b);
    return launch_depth<0, false>(depth, p, nst, out, tail_words, wgs, threads, a, b);
}

}  // namespace

// Reads each of the nbuf device buffers (bytes each, a multiple of threads x 128) in turn, reps launches in all, on
// the null stream. Launch shape: wgs work-groups of threads (64..1024) threads, depth (1..4) stages in flight (0:
// probe_fused, the read followed by partials, a barrier per half of the grid and a merge read),
// nt_policy != 0 for non-temporal loads, rr != 0 for stages dealt round robin (else one contiguous range per
// work-group; rr >= 2: round robin with the last 2 (rr - 1) rounds dealt to the odd work-groups only, a skew of rr - 1
// stages between the grid's halves), tail_bytes written by each work-group at its end. *mean_us / *best_us: the launch durations from the
// dispatch timestamps; *wall_us: the time per launch of reps launches enqueued back to back (events around them).
// Returns 0, or a HIP error code.
extern "C" int mkv_probe_run(const void* const* bufs, int nbuf, size_t bytes, int wgs, int threads, int depth,
                             int nt_policy, int rr, size_t tail_bytes, int reps, float* mean_us, float* best_us,
                             float* wall_us) {
    const size_t stage = (size_t)threads * LOADS * 16;
    const bool fused = depth <= 0;
    g_fused_mode = -depth;  // probe_fused: 512 threads, an even number of work-groups (at most 256 per half)
    if (fused && (threads != 512 || wgs % 2 || wgs > 512 || tail_bytes)) return (int)hipErrorInvalidValue;
    if (nbuf < 1 || reps < 1 || wgs < 1 || threads < 64 || threads > 1024 || threads % 64 || depth < -10 || depth > 4 ||
        bytes % stage || bytes / stage > 0xFFFFFFFFull || (tail_bytes & ~(size_t)3) % 16)
        return (int)hipErrorInvalidValue;
    // the tail's store policy rides in the low bits of tail_bytes (a multiple of 16 plus 0..3)
    g_tail_pol = (int)(tail_bytes & 3);
    // rr >= 2: round robin with a skew of rr - 1 stages between the two halves of the grid (even wgs)
    g_skew = rr >= 2 ? (unsigned)(rr - 1) : 0u;
    if (g_skew && (wgs % 2 || (size_t)g_skew * wgs >= bytes / stage)) return (int)hipErrorInvalidValue;
    tail_bytes &= ~(size_t)3;
    const unsigned nst = (unsigned)(bytes / stage), tail_words = (unsigned)(tail_bytes / 4);
    unsigned* out = nullptr;
    hipError_t e = hipMalloc(&out, (size_t)wgs * sizeof(unsigned) * (1 + tail_words) + 2 * 128 * 256);
    if (e != hipSuccess) return (int)e;
    if (fused) {
        g_epoch = 0;
        e = hipMalloc(&g_fused_part, (size_t)wgs * FUSED_PART * sizeof(float));
        if (e == hipSuccess) e = hipMalloc(&g_fused_sync, 65536 * sizeof(unsigned));
        if (e == hipSuccess) e = hipMemset(g_fused_sync, 0, 65536 * sizeof(unsigned));
        if (e == hipSuccess) e = hipMemset(out, 0, (size_t)wgs * sizeof(unsigned));
        if (e != hipSuccess) return (int)e;
    }
    hipEvent_t a, b, wa, wb;
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    (void)hipEventCreate(&wa);
    (void)hipEventCreate(&wb);
    double sum = 0.0;
    float best = 1e30f;
    for (int i = 0; i < reps && e == hipSuccess; i++) {
        e = launch_any(depth, nt_policy, rr, (const char*)bufs[i % nbuf], nst, out, tail_words, wgs, threads, a, b);
        if (e == hipSuccess) e = hipEventSynchronize(b);
        float ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
        sum += ms * 1e3;
        best = ms * 1e3f < best ? ms * 1e3f : best;
    }
    // back to back: the same launches without per-launch events, timed as a whole
    if (e == hipSuccess) e = hipEventRecord(wa, nullptr);
    for (int i = 0; i < reps && e == hipSuccess; i++)
        e = launch_any(depth, nt_policy, rr, (const char*)bufs[i % nbuf], nst, out, tail_words, wgs, threads, nullptr,
                       nullptr);
    if (e == hipSuccess) e = hipEventRecord(wb, nullptr);
    if (e == hipSuccess) e = hipEventSynchronize(wb);
    float wall = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&wall, wa, wb);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    (void)hipEventDestroy(wa);
    (void)hipEventDestroy(wb);
    if (fused && e == hipSuccess) {  // every work-group passed its barrier
        unsigned* flags = new unsigned[wgs];
        e = hipMemcpy(flags, out, (size_t)wgs * sizeof(unsigned), hipMemcpyDeviceToHost);
        for (int i = 0; i < wgs && e == hipSuccess; i++)
            if (flags[i] == 0xDEADu) e = hipErrorLaunchTimeOut;
        delete[] flags;
    }
    if (fused) {
        (void)hipFree(g_fused_part);
        (void)hipFree(g_fused_sync);
        g_fused_part = nullptr;
        g_fused_sync = nullptr;
    }
    (void)hipFree(out);
    *mean_us = (float)(sum / reps);
    *best_us = best;
    *wall_us = wall * 1e3f / reps;
    return (int)e;
}

// The bench's default read floor: 248 work-groups of 512 threads, two 64 KB stages in flight, non-temporal loads
// dealt round robin.
extern "C" int mkv_probe_read(const void* const* bufs, int nbuf, size_t bytes, int wgs, int reps, float* mean_us,
                              float* best_us) {
    float wall = 0.f;
    return mkv_probe_run(bufs, nbuf, bytes, wgs, 512, 2, 1, 1, 0, reps, mean_us, best_us, &wall);
}

// ---- the sustained rate of the f16 matrix units ----
// Every wave runs `iters` rounds of 8 independent chains of v_mfma_f32_32x32x16_f16 (register operands, nothing
// else), so the matrix units never wait on a dependence, memory or the vector units: the rate the part sustains at
// the clock it holds under that load, the ceiling the prefill kernels' MFMA fraction is read against.
namespace {
typedef _Float16 mfma_h8 __attribute__((ext_vector_type(8)));
typedef float mfma_f16v __attribute__((ext_vector_type(16)));

__global__ void __launch_bounds__(256) probe_mfma(float* __restrict__ out, int iters) {
    const int t = threadIdx.x;
    mfma_h8 a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a[i] = (_Float16)((t * 7 + i) % 13 * 0.01f);
        b[i] = (_Float16)((t * 3 + i) % 11 * 0.01f);
    }
    mfma_f16v c[8];
#pragma unroll
    for (int k = 0; k < 8; k++) c[k] = mfma_f16v{};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int k = 0; k < 8; k++) c[k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[k], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) s += c[k][0] + c[k][15];
    if (s == 1234.5f) out[blockIdx.x] = s;  // never true for these operands: keeps the chains live
}
}  // namespace

// Runs probe_mfma on wgs work-groups of 256 threads (8 per CU fill the matrix units: two waves per SIMD) for `iters`
// rounds, first for about warm_ms of back-to-back launches (the clock ramps under sustained matrix work), then reps
// timed launches. *tflops: dense f16 TFLOP/s of the timed launches (32,768 flop per MFMA); *us: their mean duration.
extern "C" int mkv_probe_mfma(int wgs, int iters, int reps, float warm_ms, float* tflops, float* us) {
    if (wgs < 1 || iters < 1 || reps < 1) return (int)hipErrorInvalidValue;
    float* out = nullptr;
    hipError_t e = hipMalloc(&out, (size_t)wgs * sizeof(float));
    if (e != hipSuccess) return (int)e;
    hipEvent_t a, b;
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    float ms = 0.f, warm = 0.f;
    while (e == hipSuccess && warm < warm_ms) {  // warm-up: launches in batches of 8 until warm_ms have passed
        e = hipEventRecord(a, nullptr);
        for (int i = 0; i < 8 && e == hipSuccess; i++) {
            hipLaunchKernelGGL(probe_mfma, dim3(wgs), dim3(256), 0, nullptr, out, iters);
            e = hipGetLastError();
        }
        if (e == hipSuccess) e = hipEventRecord(b, nullptr);
        if (e == hipSuccess) e = hipEventSynchronize(b);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
        warm += ms;
        if (ms <= 0.f) break;
    }
    if (e == hipSuccess) e = hipEventRecord(a, nullptr);
    for (int i = 0; i < reps && e == hipSuccess; i++) {
        hipLaunchKernelGGL(probe_mfma, dim3(wgs), dim3(256), 0, nullptr, out, iters);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipEventRecord(b, nullptr);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    (void)hipFree(out);
    if (e != hipSuccess) return (int)e;
    const double flop = (double)wgs * 4 * iters * 8 * 32768.0 * reps;  // 4 waves per work-group
    *us = ms * 1e3f / reps;
    *tflops = (float)(flop / (ms * 1e-3) / 1e12);
    return 0;
}
