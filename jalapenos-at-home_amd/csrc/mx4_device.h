// mx4_device.h -- device-side building blocks shared by the gfx950 kernels.
//
// MXFP4 storage (engine/src/mxfp4.rs:5-8, :27-33): weight row r of width K is
// K/2 packed bytes (element 2j in the low nibble of byte j, 2j+1 in the high
// nibble) plus K/32 E8M0 scale bytes. One 32-element block is 16 contiguous
// bytes -- exactly one 128-bit load -- and one scale byte.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mx4 {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Buffer resource over [base, base + bytes): loads past the end return zero
// without touching memory, so tail loads can be issued unconditionally.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// Greedy argmax of the logits (engine/src/model.rs:288-296: the first index of
// the maximum under a strict `>` scan from index 0) as one unsigned 64-bit key
// per row, so that the largest key is the answer: the value in an order-
// preserving integer form above the complemented row, so equal values favour
// the lower row. +0 and -0 compare equal in the scan, so both map to +0. A NaN
// is never greater than anything and nothing is greater than a NaN: a NaN at
// row 0 is the answer (key = all ones), a NaN elsewhere never is (key 0).
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t row) {
    if (v != v) return row == 0 ? ~0ull : 0ull;
    uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)b << 32) | (uint32_t)~row;
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// An f32 activation as three bf16 terms, hi + mid + lo == x, for exact
// products on the bf16 matrix cores. Each term is cut from the bits
// (truncation, never rounding up): hi keeps the top 8 significant bits of x,
// mid the top 8 of the remainder, lo what is left (at most 8 bits, exact),
// so no finite x yields an infinite term (rounding to nearest would turn
// |x| >= 0x7F7F8000 into a bf16 inf and the remainder into inf - inf = NaN).
// A non-finite x stays in hi (a NaN keeps its quiet bit in the upper half)
// with mid = lo = 0, so its products are the f32 products of the reference's
// loop: +-inf, or NaN against a zero weight.
__device__ __forceinline__ void split3_bf16(float v, __bf16& hi, __bf16& mid, __bf16& lo) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t hb = (u & 0xFFFF0000u) | (v != v ? 0x00400000u : 0u);
    float r1 = v - __uint_as_float(hb);  // NaN exactly when x is not finite
    r1 = r1 == r1 ? r1 : 0.0f;
    const uint32_t mb = __float_as_uint(r1) & 0xFFFF0000u;
    const float r2 = r1 - __uint_as_float(mb);
    hi = __builtin_bit_cast(__bf16, (uint16_t)(hb >> 16));
    mid = __builtin_bit_cast(__bf16, (uint16_t)(mb >> 16));
    lo = (__bf16)r2;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t m) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)m, off, kWave), hi = __shfl_xor((uint32_t)(m >> 32), off, kWave);
        m = max_u64(m, ((uint64_t)hi << 32) | lo);
    }
    return m;
}

// E2M1 magnitude levels (engine/src/mxfp4.rs:3).
__device__ __forceinline__ float level_of(uint32_t code) {
    // Built from bits like gpu.metal's mxfp4_level, independent of a table:
    // m = code & 7; m == 0 -> 0; m == 1 -> 0.5; else 2^(m/2 - 1) * (1 + (m & 1) / 2).
    uint32_t m = code & 7u;
    uint32_t bits = m == 0 ? 0u : (m == 1 ? 0x3f000000u : (((126u + (m >> 1)) << 23) | ((m & 1u) << 22)));
    return __uint_as_float(bits | ((code & 8u) << 28));
}

// 2^(s - 127) for an E8M0 byte s in [0, 254], exact (2^-127 is the subnormal
// 0x00400000; f32 denormals are preserved on gfx950 by default).
__device__ __forceinline__ float e8m0_to_f32(uint32_t s) {
    return __builtin_amdgcn_ldexpf(1.0f, (int)s - 127);
}

// One decoded element, bit-exact with engine/src/mxfp4.rs:27-33:
// LEVELS[c & 7] * 2^(s-127), negated when c & 8.
__device__ __forceinline__ float decode_exact(uint32_t code, uint32_t s) {
    return level_of(code) * e8m0_to_f32(s);
}

// Two E2M1 codes from byte `sel` of `word` -> two f32 levels (scale 1), using
// gfx950's hardware converter. Element order: low nibble -> .x, high -> .y.
template <int SEL>
__device__ __forceinline__ f32x2 cvt_fp4x2_f32(uint32_t word) {
    return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, SEL);
}
template <int SEL>
__device__ __forceinline__ bf16x2 cvt_fp4x2_bf16(uint32_t word) {
    return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, 1.0f, SEL);
}

__device__ __forceinline__ uint32_t as_u32(bf16x2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ bf16x2 as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2, v); }

// Sum of 32 products sum_i x[i] * level(code_i) for one MX block whose 16
// packed bytes are w (4 dwords), x given as 16 bf16 pairs in element order.
__device__ __forceinline__ float block_dot_bf16(const u32x4 w, const uint32_t* xp) {
    float acc = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        acc = __builtin_amdgcn_fdot2_f32_bf16(cvt_fp4x2_bf16<0>(w[d]), as_bf16x2(xp[4 * d + 0]), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(cvt_fp4x2_bf16<1>(w[d]), as_bf16x2(xp[4 * d + 1]), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(cvt_fp4x2_bf16<2>(w[d]), as_bf16x2(xp[4 * d + 2]), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(cvt_fp4x2_bf16<3>(w[d]), as_bf16x2(xp[4 * d + 3]), acc, false);
    }
    return acc;
}

// The same with f32 activations: products x * level are exact in f32 before
// each FMA's single rounding.
__device__ __forceinline__ float block_dot_f32(const u32x4 w, const float* x) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        f32x2 v0 = cvt_fp4x2_f32<0>(w[d]);
        f32x2 v1 = cvt_fp4x2_f32<1>(w[d]);
        f32x2 v2 = cvt_fp4x2_f32<2>(w[d]);
        f32x2 v3 = cvt_fp4x2_f32<3>(w[d]);
        a0 = __builtin_fmaf(x[8 * d + 0], v0.x, a0);
        a1 = __builtin_fmaf(x[8 * d + 1], v0.y, a1);
        a0 = __builtin_fmaf(x[8 * d + 2], v1.x, a0);
        a1 = __builtin_fmaf(x[8 * d + 3], v1.y, a1);
        a0 = __builtin_fmaf(x[8 * d + 4], v2.x, a0);
        a1 = __builtin_fmaf(x[8 * d + 5], v2.y, a1);
        a0 = __builtin_fmaf(x[8 * d + 6], v3.x, a0);
        a1 = __builtin_fmaf(x[8 * d + 7], v3.y, a1);
    }
    return a0 + a1;
}

// Wave64 sum; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ u32x4 load_u32x4(const uint8_t* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ u32x4 load_u32x4_nt(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// bf16 <-> f32 (engine/src/lib.rs:74-76 for the widening direction)
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// ---------------------------------------------------------------- LDS pipelines

// LDS barrier that does not wait for outstanding global loads (the next
// stage's prefetch stays in flight across it).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

typedef __attribute__((address_space(3))) void* lds_ptr;

// Direct-to-LDS buffer loads of 16 or 4 bytes per lane: lane l's bytes land
// at dst + l * size. (Only the device pass sees the builtin: the host pass
// checks the size against its own target, rejects 16, and would then drop
// the kernels' launch stubs without a word.)
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, lds_ptr dst, uint32_t voffset) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voffset, 0, 0, 0);
#else
    (void)r; (void)dst; (void)voffset;
#endif
}
__device__ __forceinline__ void load_lds4(__amdgpu_buffer_rsrc_t r, lds_ptr dst, uint32_t voffset) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 4, voffset, 0, 0, 0);
#else
    (void)r; (void)dst; (void)voffset;
#endif
}

}  // namespace mx4
