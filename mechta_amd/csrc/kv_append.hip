// kv_append.hip -- K/V append (RoPE + f32->f16 RNE) and conversion to / from the reference's position-major layout.
//
// Append replaces the reference's writer kernels kv_rope / kv_rope2 / kv_copy (kv.wgsl:19-42) for the f16 cache and
// rope / rope2 / copy (ops.wgsl:141-162, 275-286) for the f32 cache. One launch writes K and V of all ntok tokens:
// work items [0, nk) are K items (token, kv head, 8 dims), the rest V items (V group of positions, kv head, dim).
#include "mkv_internal.h"

namespace mkv {
namespace {

typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

template <int FMT>
__global__ void __launch_bounds__(256) append_kernel(void* __restrict__ kplane0, void* __restrict__ kplane1,
                                                     void* __restrict__ vplane0, void* __restrict__ vplane1, int pos,
                                                     int ntok, const float* __restrict__ kn,
                                                     const float* __restrict__ v, const float* __restrict__ tab,
                                                     int nk, int ng) {
    int id = blockIdx.x * blockDim.x + threadIdx.x;
    if (id < nk) {
        // K item: token t, kv head kh, dims d0..d0+7 (32 items per row)
        int t = id / (KVH * 32), kh = (id / 32) % KVH, d0 = (id % 32) * 8;
        const float* a = kn + ((size_t)t * KVH + kh) * HD;
        const float* tb = tab + (size_t)t * 64;
        float r[8];
#pragma unroll
        for (int j = 0; j < 8; j++) r[j] = rope_dim(a, tb, d0 + j);
        int p = pos + t;
        if (FMT == 0) {
            u16x8 w;
#pragma unroll
            for (int j = 0; j < 8; j++) w[j] = f2h(r[j]);
            unsigned short* kp = (unsigned short*)(kh ? kplane1 : kplane0);
            *(u16x8*)(kp + k_off(p, d0)) = w;
        } else {
            float* kp = (float*)(kh ? kplane1 : kplane0);
            *(float4*)(kp + k_off32(p, d0)) = make_float4(r[0], r[1], r[2], r[3]);
            *(float4*)(kp + k_off32(p, d0 + 4)) = make_float4(r[4], r[5], r[6], r[7]);
        }
        return;
    }
    id -= nk;
    // V item: group g (relative to the first group touched), kv head kh, dim d; a whole group is one 16-byte store
    constexpr int VG = FMT == 0 ? VGRP : VGRP32;
    if (id >= ng * KVH * HD) return;
    int gi = id / (KVH * HD), kh = (id / HD) % KVH, d = id % HD;
    int g = pos / VG + gi;
    int p0 = max(pos, g * VG), p1 = min(pos + ntok, g * VG + VG);
    const float* src = v + (size_t)kh * HD + d;  // v[t][kh*256 + d], t = p - pos
    if (FMT == 0) {
        unsigned short* vp = (unsigned short*)(kh ? vplane1 : vplane0);
        if (p0 == g * VG && p1 == g * VG + VG) {
            u16x8 w;
#pragma unroll
            for (int j = 0; j < 8; j++) w[j] = f2h(src[(size_t)(p0 + j - pos) * (KVH * HD)]);
            *(u16x8*)(vp + v_off(p0, d)) = w;
        } else {
            for (int p = p0; p < p1; p++) vp[v_off(p, d)] = f2h(src[(size_t)(p - pos) * (KVH * HD)]);
        }
    } else {
        float* vp = (float*)(kh ? vplane1 : vplane0);
        if (p0 == g * VG && p1 == g * VG + VG) {
            const size_t st = KVH * HD;
            const size_t o = (size_t)(p0 - pos) * st;
            *(float4*)(vp + v_off32(p0, d)) = make_float4(src[o], src[o + st], src[o + 2 * st], src[o + 3 * st]);
        } else {
            for (int p = p0; p < p1; p++) vp[v_off32(p, d)] = src[(size_t)(p - pos) * (KVH * HD)];
        }
    }
}

// Position-major <-> store layout for [p0, p1) of one (layer, K|V): element (pos, kvh, d) of the reference layout
// at ((pos - p0)*2 + kvh)*256 + d.
template <typename T, int DIR>  // DIR 0: store -> rows, 1: rows -> store
__global__ void __launch_bounds__(256) rows_kernel(T* __restrict__ plane0, T* __restrict__ plane1,
                                                   T* __restrict__ rows, int p0, int p1, int which, int fmt) {
    size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t total = (size_t)(p1 - p0) * KVH * HD;
    if (id >= total) return;
    int d = id % HD, kh = (id / HD) % KVH, p = p0 + (int)(id / (KVH * HD));
    T* plane = kh ? plane1 : plane0;
    size_t o = fmt == 1 ? (which == 0 ? k_off32(p, d) : v_off32(p, d)) : (which == 0 ? k_off(p, d) : v_off(p, d));
    if (DIR == 0) rows[id] = plane[o];
    else plane[o] = rows[id];
}

}  // namespace

hipError_t launch_append(const Geom& g, void* base, int layer, int pos, int ntok, const float* kn, const float* v,
                         const float* tab, const Launch& L) {
    char* b = (char*)base;
    void* k0 = b + g.plane(layer, 0, 0) * g.plane_bytes();
    void* k1 = b + g.plane(layer, 0, 1) * g.plane_bytes();
    void* v0 = b + g.plane(layer, 1, 0) * g.plane_bytes();
    void* v1 = b + g.plane(layer, 1, 1) * g.plane_bytes();
    int nk = ntok * KVH * 32;
    const int vg = plane_unit(g.fmt, 1);
    int ng = (pos + ntok - 1) / vg - pos / vg + 1;
    int nv = ng * KVH * HD;
    int blocks = (nk + nv + 255) / 256;
    return launch(g.fmt == 0 ? append_kernel<0> : append_kernel<1>, dim3(blocks), dim3(256), L, k0, k1, v0, v1, pos,
                  ntok, kn, v, tab, nk, ng);
}

static hipError_t launch_rows(const Geom& g, const void* base, int layer, int which, int p0, int p1, void* rows,
                              int dir, const Launch& L) {
    char* b = (char*)base;
    void* q0 = b + g.plane(layer, which, 0) * g.plane_bytes();
    void* q1 = b + g.plane(layer, which, 1) * g.plane_bytes();
    size_t total = (size_t)(p1 - p0) * KVH * HD;
    if (total == 0) return hipSuccess;
    unsigned blocks = (unsigned)((total + 255) / 256);
    if (g.fmt == 0)
        return launch(dir == 0 ? rows_kernel<unsigned short, 0> : rows_kernel<unsigned short, 1>, dim3(blocks),
                      dim3(256), L, q0, q1, rows, p0, p1, which, 0);
    return launch(dir == 0 ? rows_kernel<float, 0> : rows_kernel<float, 1>, dim3(blocks), dim3(256), L, q0, q1, rows,
                  p0, p1, which, 1);
}

hipError_t launch_read_rows(const Geom& g, const void* base, int layer, int which, int p0, int p1, void* dst,
                            const Launch& L) {
    return launch_rows(g, base, layer, which, p0, p1, dst, 0, L);
}

hipError_t launch_write_rows(const Geom& g, void* base, int layer, int which, int p0, int p1, const void* src,
                             const Launch& L) {
    return launch_rows(g, base, layer, which, p0, p1, const_cast<void*>(src), 1, L);
}

}  // namespace mkv
