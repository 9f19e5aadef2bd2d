// mkv_device.h -- device helpers shared by the attention kernels (gfx950).
#pragma once
#include "mkv_internal.h"

namespace mkv {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LAZY2 = 8.0f * LOG2E;  // DM_LAZY = 8 (dmx.rs:124) in log2 units
constexpr float NEG_INF = -__builtin_huge_valf();

// 2^x with the hardware's v_exp_f32 (no denormal scaffolding: results below 2^-126 flush to 0, far below the
// smallest f16 P of 2^-24).
__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline f32x16 mfma32(half8 a, half8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ inline f32x4 mfma16(half8 a, half8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// f32 products on the f16 matrix units. An f32 operand x is split into two f16 parts: hi = f16(x), rounded to nearest
// even, and lo = f16(x - hi) (the difference is exact in f32), so |x - hi| <= 2^-11 |x| and |x - hi - lo| <= 2^-22 |x|
// for |x| in f16's normal range. Per pair of elements: one packed conversion for hi, two v_fma_mix_f32 for x - hi (the
// f16 hi read from its half of the packed register, so no conversion back to f32), one packed conversion for lo: two
// vector instructions per element (clearing hi's low mantissa bits with an AND, then a subtraction, took three). A
// product a.b is taken as hi(a)hi(b) + hi(a)lo(b) + lo(a)hi(b) with f32 accumulation; the dropped lo(a)lo(b) is below
// 2^-22 of |a||b|. Operands that are f16 already (an f16 cache's K or V) need two passes. The inputs of a split are
// never MFMA results read directly (inline assembly gets no hazard wait states from the compiler): they are loads, or
// the softmax's vector results.
template <bool HIGH>  // x - (float)(the f16 in the low or high half of pair)
__device__ inline float sub_half(float x, unsigned pair) {
    float d;
    if constexpr (HIGH)
        asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(pair), "v"(x));
    else
        asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(pair), "v"(x));
    return d;
}
__device__ inline void split2(float a, float b, unsigned& hi, unsigned& lo) {
    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    const half2v h = {(_Float16)a, (_Float16)b};
    hi = __builtin_bit_cast(unsigned, h);
    const half2v l = {(_Float16)sub_half<false>(a, hi), (_Float16)sub_half<true>(b, hi)};
    lo = __builtin_bit_cast(unsigned, l);
}
__device__ inline void split8(f32x4 a, f32x4 b, half8& hi, half8& lo) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    unsigned h0, h1, h2, h3, l0, l1, l2, l3;
    split2(a.x, a.y, h0, l0);
    split2(a.z, a.w, h1, l1);
    split2(b.x, b.y, h2, l2);
    split2(b.z, b.w, h3, l3);
    hi = __builtin_bit_cast(half8, u32x4{h0, h1, h2, h3});
    lo = __builtin_bit_cast(half8, u32x4{l0, l1, l2, l3});
}
// c += a.b with a = ah + al, b = bh + bl: three f16 MFMAs (al.bl dropped)
__device__ inline f32x16 mfma3(half8 ah, half8 al, half8 bh, half8 bl, f32x16 c) {
    c = mfma32(ah, bh, c);
    c = mfma32(ah, bl, c);
    return mfma32(al, bh, c);
}
__device__ inline void split4(f32x4 a, half4& hi, half4& lo) {
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    unsigned h0, h1, l0, l1;
    split2(a.x, a.y, h0, l0);
    split2(a.z, a.w, h1, l1);
    hi = __builtin_bit_cast(half4, u32x2{h0, h1});
    lo = __builtin_bit_cast(half4, u32x2{l0, l1});
}
// c += a.(bh + bl) with a exact in f16: two passes
__device__ inline f32x16 mfma2(half8 a, half8 bh, half8 bl, f32x16 c) { return mfma32(a, bl, mfma32(a, bh, c)); }
__device__ inline f32x4 mfma16k32(half8 a, half8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ inline f32x4 mfma16k16(half4 a, half4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Key offset inside a 32-key K block of the key loaded by A-operand row m of the 32x32 MFMA. The C layout of that
// MFMA gives lane half h the rows 8a + 4h + b (register 4a + b); loading row m from key perm(m) makes register i of
// lane half h hold key 8h + i (i < 8) or 16 + 8h + (i - 8) (i >= 8): exactly the keys the A operand (P) of the
// following P.V MFMA needs in that lane, so S^T = K.Q^T turns into P without leaving the registers.
__device__ inline int key_perm(int m) {
    int a = m >> 3, c = (m >> 2) & 1, b = m & 3;
    return 16 * (a >> 1) + 8 * c + 4 * (a & 1) + b;
}

// Reduction over the 16 lanes of a DPP row: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror
// (lane swaps inside the ALU, no LDS round trip).
template <typename Op>
__device__ inline float reduce16(float x, Op op) {
    x = op(x, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, true)));
    x = op(x, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, true)));
    x = op(x, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x141, 0xF, 0xF, true)));
    x = op(x, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x140, 0xF, 0xF, true)));
    return x;
}

// Raw buffer access: a 16-byte load whose offset lies past the resource's `bytes` returns zeros without a memory
// access, which masks lanes or whole loads without a branch (and so without the waits a branch around a load makes
// the compiler insert).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
// base and bytes must be wave-uniform; they are read from the first lane so that the resource lives in scalar
// registers (a resource in vector registers makes the compiler loop over lanes around every load)
__device__ inline rsrc_t plane_rsrc(const void* base, unsigned bytes) {
    const unsigned long long a = (unsigned long long)base;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)a), hi = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32));
    void* b = (void*)(((unsigned long long)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(b, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
// Cache policy of the K/V plane loads. The planes are read once per launch: loaded non-temporal (policy bit nt = 2),
// the streamed planes do not displace other lines (measured per launch from HBM: f16 decode 25.0 against 26.0 us,
// f32 decode about 1 us less, Flint f32 decode 32 against 34 us).
constexpr int LOAD_NT = 2;
// Policy bit sc1 (16): a device-coherent load, for split partials another work-group of the same launch stored with
// agent-scope atomic stores (the fused merges of the decodes).
constexpr int LOAD_SC1 = 16;
__device__ inline half8 bload16(rsrc_t r, unsigned off) {
    return __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, LOAD_NT));
}

// Work-group barrier for LDS traffic only: waits for this wave's LDS operations, not for its global loads (a
// __syncthreads() would also wait for every pending global load and drain the loads already in flight).
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Direct global -> LDS load of 64 lanes x 16 bytes: lane i's 16 bytes from src land at lds_base + 16i. Issued as
// inline assembly, so the compiler neither counts it nor orders LDS reads behind it: every wait for these loads is
// an explicit s_waitcnt in the caller (the compiler's own waits for its loads stay correct, they only wait longer).
__device__ inline void dma16(const void* src, void* lds_base) {
    const unsigned lds = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_void*)lds_base);  // wave-uniform
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}
// The same load with a wave-uniform 64-bit base in scalar registers and a 32-bit per-lane byte offset (the
// instruction's saddr form): lane i's 16 bytes from sbase + voff land at lds + 16i. With the base and the LDS address
// computed on the scalar unit, issuing a tile's loads takes no vector instruction.
// Both helpers set m0, which the compiler reserves (hipcc warns about a reserved register in the clobber list): the
// generated code of these kernels holds no value of its own in m0 (no LDS-DMA builtin, no s_sendmsg, no relative
// VGPR indexing), so nothing live is overwritten. __builtin_amdgcn_global_load_lds manages m0 itself, but for these
// loads it builds 64-bit per-lane addresses (8 more vector instructions per prefill_f16 tile and wave): measured, the
// cfg3 prefill fell from 43.7% to 42.0% of the f16 peak and the f32 prefill rose from 0.453 to 0.464 ms.
__device__ inline void dma16s(const void* sbase, unsigned voff, unsigned lds) {
    // both halves of the base through readfirstlane: scalar registers whatever the compiler proved (free when it did);
    // readfirstlane returns int, so each half widens through unsigned (no sign extension into the high word)
    const unsigned long long a = (unsigned long long)(uintptr_t)sbase;
    const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((unsigned)(a >> 32));
    const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((unsigned)a);
    const unsigned long long b = (unsigned long long)hi << 32 | lo;
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(b),
                 "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory", "m0");
}


// Maxima of the softmax on scores that are never NaN (masked scores are -inf), as single instructions: fmaxf's NaN
// handling would add a canonicalizing max per operand. Inline assembly gets no hazard wait states from the compiler:
// its operands must not be MFMA results read directly (a vector read of those needs wait states the compiler inserts
// only before its own instructions), so a chain over accumulators starts with a compiler maximum.
__device__ inline float vmax(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ inline float vmax3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
// The maximum over lanes l and l ^ 32, in every lane: v_permlane32_swap of two registers that both hold x leaves one
// half's values in both halves of one register and the other half's in the other (the copy makes them two registers:
// with one register the swap would exchange a register's halves with themselves).
__device__ inline float max_xor32(float x) {
    float y;
    asm volatile("v_mov_b32 %0, %1" : "=v"(y) : "v"(x));
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// The sum over lanes l and l ^ 32, in every lane (the same two registers; a + b == b + a, so every lane holds what
// x + __shfl_xor(x, 32) would give)
__device__ inline float add_xor32(float x) {
    float y;
    asm volatile("v_mov_b32 %0, %1" : "=v"(y) : "v"(x));
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace mkv
