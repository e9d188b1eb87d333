// quant.hip -- MXFP4 format kernels: quantize (the weight recipe and the
// activation requantizer of the MFMA path), MX-FP8 requantize, dequantize,
// first-max argmax, scale range scan and the synthetic-input generator.
#include <type_traits>

#include "mx_encode.h"
#include "mx4_device.h"
#include "mx4_kernels.h"

namespace mx4 {

// ------------------------------------------------------------------ quantize

// python/quantize_mxfp4.py:18-39 for one 32-element block. The scale byte is
// s = max(E - 2, 0) with E the biased exponent of amax (0 for zero or
// subnormal amax): frexp(amax).exp - 3 = E - 129, clipped at -127.
// Largest |v| of a block and whether every value is finite, as a tree over
// the magnitude bits (for non-negative floats the bit patterns order like the
// values, so the maximum is exact in any order; a tree keeps the dependency
// chain at 5 steps instead of 32). `finite` is false for inf and NaN.
__device__ __forceinline__ float block_amax(const float (&v)[32], bool& finite) {
    uint32_t m[16], e[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t a = __float_as_uint(v[i]) & 0x7fffffffu, b = __float_as_uint(v[i + 16]) & 0x7fffffffu;
        m[i] = a > b ? a : b;
        e[i] = ((a & 0x7f800000u) == 0x7f800000u) | ((b & 0x7f800000u) == 0x7f800000u);
    }
#pragma unroll
    for (int w = 8; w >= 1; w /= 2)
#pragma unroll
        for (int i = 0; i < w; ++i) {
            m[i] = m[i] > m[i + w] ? m[i] : m[i + w];
            e[i] |= e[i + w];
        }
    finite = e[0] == 0;
    return __uint_as_float(m[0]);
}

__device__ __forceinline__ uint32_t mxfp4_scale_byte(float amax) {
    int e_biased = (int)((__float_as_uint(amax) >> 23) & 0xffu);
    int s = e_biased - 2;
    return s < 0 ? 0u : (uint32_t)s;
}

__device__ __forceinline__ uint32_t mxfp4_code(float v, uint32_t s) {
    const float scaled = __builtin_amdgcn_ldexpf(__builtin_fabsf(v), 127 - (int)s);
    return e2m1_magnitude_code(scaled) | ((__float_as_uint(v) >> 31) << 3);  // signbit, so -0.0 -> code 8
}

template <bool BF16>
__device__ __forceinline__ void load_block32(const void* in, uint64_t blk, float (&v)[32]) {
    if constexpr (BF16) {
        const uint8_t* p = static_cast<const uint8_t*>(in) + blk * 64;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            u32x4 w = load_u32x4(p + 16 * q);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                v[8 * q + 2 * c] = bf16_bits_to_f32(w[c] & 0xffffu);
                v[8 * q + 2 * c + 1] = bf16_bits_to_f32(w[c] >> 16);
            }
        }
    } else {
        const float* p = static_cast<const float*>(in) + blk * 32;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            f32x4 w = *reinterpret_cast<const f32x4*>(p + 4 * q);
            v[4 * q + 0] = w[0];
            v[4 * q + 1] = w[1];
            v[4 * q + 2] = w[2];
            v[4 * q + 3] = w[3];
        }
    }
}

// One thread per 32-element block (blocks are consecutive in memory, so
// block b of the flat tensor is row b / (cols/32), column block b % (cols/32)).
template <bool BF16>
__global__ __launch_bounds__(256) void quantize_mxfp4_kernel(const void* __restrict__ in, uint64_t blocks,
                                                             uint8_t* __restrict__ packed,
                                                             uint8_t* __restrict__ scales,
                                                             uint32_t* __restrict__ bad) {
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    float v[32];
    load_block32<BF16>(in, b, v);
    bool finite;
    const float amax = block_amax(v, finite);
    if (!finite) atomicOr(bad, 1u);
    const uint32_t s = mxfp4_scale_byte(amax);
    u32x4 out;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) word |= mxfp4_code(v[8 * d + i], s) << (4 * i);
        out[d] = word;
    }
    *reinterpret_cast<u32x4*>(packed + b * 16) = out;
    scales[b] = (uint8_t)s;
}

hipError_t launch_quantize_mxfp4(const void* in, bool in_bf16, uint64_t rows, uint32_t cols,
                                 uint8_t* packed, uint8_t* scales, uint32_t* bad, hipStream_t s) {
    const uint64_t blocks = rows * (cols / 32);
    if (blocks == 0) return hipSuccess;
    dim3 grid((unsigned)((blocks + 255) / 256));
    if (in_bf16)
        hipLaunchKernelGGL(quantize_mxfp4_kernel<true>, grid, dim3(256), 0, s, in, blocks, packed, scales, bad);
    else
        hipLaunchKernelGGL(quantize_mxfp4_kernel<false>, grid, dim3(256), 0, s, in, blocks, packed, scales, bad);
    return hipGetLastError();
}

// MX-FP8 E4M3: e = floor(log2 amax) - 8 clipped to [-127, 127], RNE onto the
// E4M3 grid, saturating at 448 (code 0x7e).
__device__ __forceinline__ uint32_t fp8_scale_byte(float amax) {
    int e_biased = (int)((__float_as_uint(amax) >> 23) & 0xffu);
    // normal amax: floor(log2) = E - 127, e = E - 135, s = E - 8
    int s = e_biased - 8;
    return s < 0 ? 0u : (uint32_t)s;
}

__device__ __forceinline__ uint32_t e4m3_code(float v, uint32_t s) {
    const float scaled = __builtin_amdgcn_ldexpf(__builtin_fabsf(v), 127 - (int)s);
    return e4m3_magnitude_code(scaled) | ((__float_as_uint(v) >> 31) << 7);
}

template <bool BF16>
__global__ __launch_bounds__(256) void quantize_fp8_kernel(const void* __restrict__ in, uint64_t blocks,
                                                           uint8_t* __restrict__ codes,
                                                           uint8_t* __restrict__ scales,
                                                           uint32_t* __restrict__ bad) {
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    float v[32];
    load_block32<BF16>(in, b, v);
    bool finite;
    const float amax = block_amax(v, finite);
    if (!finite) atomicOr(bad, 1u);
    const uint32_t s = fp8_scale_byte(amax);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        u32x4 out;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) word |= e4m3_code(v[16 * q + 4 * d + i], s) << (8 * i);
            out[d] = word;
        }
        *reinterpret_cast<u32x4*>(codes + b * 32 + 16 * q) = out;
    }
    scales[b] = (uint8_t)s;
}

hipError_t launch_quantize_fp8(const void* in, bool in_bf16, uint64_t rows, uint32_t cols,
                               uint8_t* codes, uint8_t* scales, uint32_t* bad, hipStream_t s) {
    const uint64_t blocks = rows * (cols / 32);
    if (blocks == 0) return hipSuccess;
    dim3 grid((unsigned)((blocks + 255) / 256));
    if (in_bf16)
        hipLaunchKernelGGL(quantize_fp8_kernel<true>, grid, dim3(256), 0, s, in, blocks, codes, scales, bad);
    else
        hipLaunchKernelGGL(quantize_fp8_kernel<false>, grid, dim3(256), 0, s, in, blocks, codes, scales, bad);
    return hipGetLastError();
}

// Fragment-native output (prefill.hip): the same rules as above. A workgroup
// of four waves takes row group g and J consecutive k-steps (32 rows x 64 J
// columns; J = 4: a whole scale quad). Thread i works on row 32 g + i / 8 and,
// in each of its J k-steps, on the 8 consecutive values [8 p, +8) of the
// k-step (p = i % 8): it issues the J k-steps' loads before it uses any, and
// each wave's load of one k-step covers whole row spans (one 128-byte line
// per row for bf16). The four threads of a 32-element block (p in 0..3
// or 4..7: block h = p / 4 of the k-step) meet in a DPP max for its scale;
// each encodes its 8 values and stores them where the fragment holds them:
// FP4 bytes [4 (p % 4), +4) of lane r32 + 32 h's 16, FP8 the 8 bytes of K
// [8 p, +8) (lane group (p % 4) / 2 of KiB h). The block's first thread holds
// the J k-steps' scale bytes of lane r32 + 32 h and stores them together:
// bytes kk % 4 .. kk % 4 + J - 1 of that lane's word of quad kk / 4. Rows past `rows` in the last group are written as
// zero codes and scales; a block with a non-finite value gets scale byte 0xff
// (E8M0 NaN), so its products -- and the row's outputs -- are NaN instead of
// finite values of a meaningless scale.
template <bool BF16, bool FP8, int J>
__global__ __launch_bounds__(256) void quantize_fragments_kernel(const void* __restrict__ in, uint32_t rows,
                                                                 uint32_t cols, uint8_t* __restrict__ codes,
                                                                 uint8_t* __restrict__ scales,
                                                                 uint32_t* __restrict__ bad) {
    static_assert(J == 1 || J == 2 || J == 4, "k-steps per workgroup: 1, 2 or 4 (a whole scale quad)");
    using SW = std::conditional_t<J == 4, uint32_t, std::conditional_t<J == 2, uint16_t, uint8_t>>;
    constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E;  // DPP quad_perm [1,0,3,2], [2,3,0,1]
    const uint32_t t = threadIdx.x, p = t % 8, r32 = t / 8, h = p / 4;
    const uint32_t nk = cols / 64, nq = cols / 256;
    const uint32_t nb = nk / J, b = blockIdx.x % nb, g = blockIdx.x / nb;  // k-steps [J b, J b + J)
    const uint32_t row = 32 * g + r32;
    float v[J][8];
    if (row < rows) {
        const uint64_t e0 = (uint64_t)row * cols + 64 * J * b + 8 * p;
        if constexpr (BF16) {
            u32x4 w[J];
#pragma unroll
            for (int j = 0; j < J; ++j) w[j] = load_u32x4(static_cast<const uint8_t*>(in) + 2 * (e0 + 64 * j));
#pragma unroll
            for (int j = 0; j < J; ++j)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    v[j][2 * c] = bf16_bits_to_f32(w[j][c] & 0xffffu);
                    v[j][2 * c + 1] = bf16_bits_to_f32(w[j][c] >> 16);
                }
        } else {
            f32x4 a[J], bq[J];
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const f32x4* src = reinterpret_cast<const f32x4*>(static_cast<const float*>(in) + e0 + 64 * j);
                a[j] = src[0];
                bq[j] = src[1];
            }
#pragma unroll
            for (int j = 0; j < J; ++j)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    v[j][c] = a[j][c];
                    v[j][4 + c] = bq[j][c];
                }
        }
    } else {
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) v[j][i] = 0.0f;
    }
    uint32_t sword = 0, any_bad = 0;  // the scale bytes of k-steps J b .. J b + J - 1
#pragma unroll
    for (int j = 0; j < J; ++j) {
        // the block's largest magnitude, as bits (non-negative floats order
        // like their bit patterns, so the maximum is exact in any order), and
        // whether any value is inf or NaN
        uint32_t mx = 0, nonfinite = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t a = __float_as_uint(v[j][i]) & 0x7fffffffu;
            mx = a > mx ? a : mx;
            nonfinite |= a >= 0x7f800000u ? 1u : 0u;
        }
        {
            uint32_t om = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mx, kQuadXor1, 0xF, 0xF, false);
            nonfinite |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)nonfinite, kQuadXor1, 0xF, 0xF, false);
            mx = om > mx ? om : mx;
            om = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mx, kQuadXor2, 0xF, 0xF, false);
            nonfinite |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)nonfinite, kQuadXor2, 0xF, 0xF, false);
            mx = om > mx ? om : mx;
        }
        const float amax = __uint_as_float(mx);
        const bool finite = nonfinite == 0;
        any_bad |= nonfinite;
        const uint64_t frag = (uint64_t)g * nk + J * b + j;
        uint32_t s;
        if constexpr (FP8) {
            s = fp8_scale_byte(amax);
            uint32_t w0 = 0, w1 = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                w0 |= e4m3_code(v[j][i], s) << (8 * i);
                w1 |= e4m3_code(v[j][4 + i], s) << (8 * i);
            }
            uint8_t* dst = codes + frag * 2048 + h * 1024 + (32 * ((p % 4) / 2) + r32) * 16 + 8 * (p % 2);
            *reinterpret_cast<uint2*>(dst) = make_uint2(w0, w1);
        } else {
            s = mxfp4_scale_byte(amax);
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) word |= mxfp4_code(v[j][i], s) << (4 * i);
            *reinterpret_cast<uint32_t*>(codes + (frag * 64 + r32 + 32 * h) * 16 + 4 * (p % 4)) = word;
        }
        sword |= (finite ? s : 0xffu) << (8 * j);
    }
    if (p % 4 == 0) {
        if (any_bad) atomicOr(bad, 1u);
        // byte kk % 4 of lane r32 + 32 h's word of quad kk / 4, for J k-steps at once
        const uint32_t kk = J * b;
        reinterpret_cast<SW*>(scales + (((uint64_t)g * nq + kk / 4) * 64 + r32 + 32 * h) * 4 + kk % 4)[0] = (SW)sword;
    }
}

hipError_t launch_quantize_fragments(const void* in, bool in_bf16, uint32_t rows, uint32_t cols, bool fp8,
                                     uint8_t* codes_f, uint8_t* scales_f, uint32_t* bad, hipStream_t s) {
    if (rows == 0 || cols == 0) return hipSuccess;
    if (cols % 256 != 0) return hipErrorInvalidValue;
    // A whole scale quad per workgroup on wide rows, one k-step on narrower
    // ones (more waves per SIMD to overlap the encode). bf16 512 x 12288, in
    // a recorded pass: 7.10 / 7.05 -> 6.80 / 6.63 us per call (MXFP4 /
    // MX-FP8); at 512 x 4096 the one-k-step form measured 4.17-4.30 us
    // against 4.31-4.45 for whole quads (two k-steps: slower than either).
    auto go = [&](auto j_tag) {
        constexpr int J = decltype(j_tag)::value;
        const uint64_t wgs = (uint64_t)((rows + 31) / 32) * (cols / (64 * J));
        if (wgs > 0x7fffffffu) return hipErrorInvalidValue;
        dim3 grid((unsigned)wgs);
        if (in_bf16) {
            if (fp8)
                hipLaunchKernelGGL((quantize_fragments_kernel<true, true, J>), grid, dim3(256), 0, s, in, rows, cols,
                                   codes_f, scales_f, bad);
            else
                hipLaunchKernelGGL((quantize_fragments_kernel<true, false, J>), grid, dim3(256), 0, s, in, rows, cols,
                                   codes_f, scales_f, bad);
        } else {
            if (fp8)
                hipLaunchKernelGGL((quantize_fragments_kernel<false, true, J>), grid, dim3(256), 0, s, in, rows, cols,
                                   codes_f, scales_f, bad);
            else
                hipLaunchKernelGGL((quantize_fragments_kernel<false, false, J>), grid, dim3(256), 0, s, in, rows,
                                   cols, codes_f, scales_f, bad);
        }
        return hipGetLastError();
    };
    return cols >= 8192 ? go(std::integral_constant<int, 4>{}) : go(std::integral_constant<int, 1>{});
}

// ------------------------------------------------------------------ embedding

// engine/src/lib.rs:222-227 (embed): row ids[t] of the table, each value
// decoded exactly (engine/src/mxfp4.rs:35-49) and cut to bf16 by dropping the
// low 16 bits, as both the CPU path (`to_bits() >> 16`) and the Metal kernel
// (engine/src/gpu.metal:43-55, `& 0xffff0000`) do. One thread per 32 values.
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t* __restrict__ packed, const uint8_t* __restrict__ scales,
                                                    const uint16_t* __restrict__ bf16, const uint32_t* __restrict__ ids,
                                                    uint32_t count, uint32_t rows, uint32_t cols,
                                                    uint16_t* __restrict__ out) {
    const uint32_t nblk = cols / 32;
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (uint64_t)count * nblk) return;
    const uint32_t tok = (uint32_t)(t / nblk), b = (uint32_t)(t % nblk);
    const uint32_t id = ids[tok];
    uint32_t words[16];
    if (id >= rows) {
#pragma unroll
        for (int i = 0; i < 16; ++i) words[i] = 0;
    } else if (bf16) {
        const u32x4* src = reinterpret_cast<const u32x4*>(bf16 + (uint64_t)id * cols + 32 * (uint64_t)b);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 v = src[q];
#pragma unroll
            for (int e = 0; e < 4; ++e) words[4 * q + e] = v[e];
        }
    } else {
        const u32x4 w = load_u32x4(packed + ((uint64_t)id * nblk + b) * 16);
        const uint32_t s = scales[(uint64_t)id * nblk + b];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t byte = (w[e / 4] >> (8 * (e % 4))) & 0xffu;
            const uint32_t lo = __float_as_uint(decode_exact(byte & 15u, s)) >> 16;
            const uint32_t hi = __float_as_uint(decode_exact(byte >> 4, s)) >> 16;
            words[e] = lo | (hi << 16);
        }
    }
    u32x4* dst = reinterpret_cast<u32x4*>(out + (uint64_t)tok * cols + 32 * (uint64_t)b);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = u32x4{words[4 * q], words[4 * q + 1], words[4 * q + 2], words[4 * q + 3]};
}

hipError_t launch_embed(const uint8_t* packed, const uint8_t* scales, const uint16_t* bf16, const uint32_t* ids,
                        uint32_t count, uint32_t rows, uint32_t cols, uint16_t* out, hipStream_t s) {
    const uint64_t threads = (uint64_t)count * (cols / 32);
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, packed, scales, bf16, ids,
                       count, rows, cols, out);
    return hipGetLastError();
}

// ------------------------------------------------------------------ dequantize

// engine/src/mxfp4.rs:35-49: one thread per packed byte -> two f32 values.
__global__ __launch_bounds__(256) void dequantize_kernel(const uint8_t* __restrict__ packed,
                                                         const uint8_t* __restrict__ scales,
                                                         uint64_t bytes, float* __restrict__ out) {
    const uint64_t j = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= bytes) return;
    const uint32_t byte = packed[j];
    const uint32_t s = scales[j / 16];
    f32x2 v;
    v.x = decode_exact(byte & 15u, s);
    v.y = decode_exact(byte >> 4, s);
    *reinterpret_cast<f32x2*>(out + 2 * j) = v;
}

hipError_t launch_dequantize(const uint8_t* packed, const uint8_t* scales, uint64_t elements,
                             float* out, hipStream_t s) {
    const uint64_t bytes = elements / 2;
    if (bytes == 0) return hipSuccess;
    hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)((bytes + 255) / 256)), dim3(256), 0, s, packed,
                       scales, bytes, out);
    return hipGetLastError();
}

// Decode tables for the exhaustive converter check: out[s * 16 + c].
//  mode 0: decode_exact (bit construction x ldexp)
//  mode 1: hardware fp4 -> f32 at scale 1, times 2^(s-127) (the GEMV factorisation)
//  mode 2: hardware fp4 -> bf16 with the scale folded in, widened to f32
//  mode 3: hardware fp4 -> f32 with the scale folded in
__global__ void decode_table_kernel(int mode, float* out) {
    const uint32_t s = blockIdx.x;      // 0..255
    const uint32_t c = threadIdx.x;     // 0..15
    const uint32_t word = c | (c << 4); // byte 0 holds the code in both nibbles
    float v;
    if (mode == 0) {
        v = decode_exact(c, s);
    } else if (mode == 1) {
        v = cvt_fp4x2_f32<0>(word).x * e8m0_to_f32(s);
    } else if (mode == 2) {
        bf16x2 p = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, e8m0_to_f32(s), 0);
        v = bf16_bits_to_f32(as_u32(p) & 0xffffu);
    } else {
        v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, e8m0_to_f32(s), 0)[0];
    }
    out[s * 16 + c] = v;
}

hipError_t launch_decode_table(int mode, float* out, hipStream_t s) {
    hipLaunchKernelGGL(decode_table_kernel, dim3(256), dim3(16), 0, s, mode, out);
    return hipGetLastError();
}

// Smallest and largest scale byte (out2[0] = min, out2[1] = max); out2 must
// start at {255, 0}.
__global__ __launch_bounds__(256) void min_max_scale_kernel(const uint8_t* __restrict__ scales,
                                                            uint64_t count, uint32_t* out2) {
    uint32_t lo = 255, hi = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t v = scales[i];
        lo = v < lo ? v : lo;
        hi = v > hi ? v : hi;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        uint32_t a = __shfl_xor(lo, off, 64), b = __shfl_xor(hi, off, 64);
        lo = a < lo ? a : lo;
        hi = b > hi ? b : hi;
    }
    if (threadIdx.x % 64 == 0) {
        atomicMin(out2, lo);
        atomicMax(out2 + 1, hi);
    }
}

hipError_t launch_min_max_scale(const uint8_t* scales, uint64_t count, uint32_t* out2, hipStream_t s) {
    uint64_t groups = (count + 255) / 256;
    if (groups > 2048) groups = 2048;
    if (groups == 0) groups = 1;
    hipLaunchKernelGGL(min_max_scale_kernel, dim3((unsigned)groups), dim3(256), 0, s, scales, count, out2);
    return hipGetLastError();
}

// ------------------------------------------------------------------ argmax

// engine/src/model.rs:288-296 per row: the first index of the maximum under a
// strict `>` scan from column 0, so a NaN never wins unless it sits in column 0
// (nothing compares greater than it), and ties go to the lowest index. Row r is
// cut into `chunks` pieces of `chunk` columns; block (r, c) reduces its piece to
// one argmax_key. A thread scans its columns in increasing order with a strict
// `>` (first maximum within the thread); keys order the threads and blocks.
// With one chunk per row the block writes the index; otherwise its key goes to
// partial[r * chunks + c] for argmax_reduce_kernel. Each trip issues four
// unconditional loads per thread (4 KiB per block in flight) through a buffer
// resource bounded to the piece; loads past its end return zero and are masked.
template <bool FINAL>
__global__ __launch_bounds__(256) void argmax_chunk_kernel(const float* __restrict__ x, uint32_t width,
                                                           uint32_t chunk, uint32_t chunks,
                                                           uint64_t* __restrict__ partial, uint32_t* __restrict__ out) {
    const uint32_t row = blockIdx.x / chunks, c = blockIdx.x % chunks;
    const uint32_t start = c * chunk;  // < width: the host makes every piece non-empty
    const uint32_t len = min(chunk, width - start);
    const float* base = x + (size_t)row * width + start;
    const __amdgpu_buffer_rsrc_t r = rsrc(base, len * 4u);
    float best = -__builtin_inff();
    uint32_t at = 0xffffffffu;
    for (uint32_t i = threadIdx.x; i < len; i += 256 * 4) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, 4 * (i + 256 * j), 0, 0));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (i + 256 * j < len && v[j] > best) {
                best = v[j];
                at = i + 256 * j;
            }
        }
    }
    uint64_t key = at == 0xffffffffu ? 0ull : argmax_key(best, start + at);
    if (c == 0 && threadIdx.x == 0 && base[0] != base[0]) key = ~0ull;  // NaN in column 0
    key = wave_max_u64(key);
    __shared__ uint64_t wm[4];
    if (threadIdx.x % 64 == 0) wm[threadIdx.x / 64] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        key = max_u64(max_u64(wm[0], wm[1]), max_u64(wm[2], wm[3]));
        if constexpr (FINAL) {
            out[row] = key == 0 ? 0u : ~(uint32_t)key;  // key 0: no candidate (all -inf or NaN) -> column 0
        } else {
            partial[blockIdx.x] = key;
        }
    }
}

// Block r reduces the `count` keys partial[r * count ..] of row r to its index.
__global__ __launch_bounds__(256) void argmax_reduce_kernel(const uint64_t* __restrict__ partial, uint32_t count,
                                                            uint32_t* __restrict__ out) {
    const uint64_t* p = partial + (size_t)blockIdx.x * count;
    uint64_t m = 0;
    for (uint32_t i = threadIdx.x; i < count; i += 256) m = max_u64(m, p[i]);
    m = wave_max_u64(m);
    __shared__ uint64_t wm[4];
    if (threadIdx.x % 64 == 0) wm[threadIdx.x / 64] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = max_u64(max_u64(wm[0], wm[1]), max_u64(wm[2], wm[3]));
        out[blockIdx.x] = m == 0 ? 0u : ~(uint32_t)m;
    }
}

hipError_t launch_argmax_reduce(const uint64_t* partial, uint32_t rows, uint32_t count, uint32_t* out, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(argmax_reduce_kernel, dim3(rows), dim3(256), 0, s, partial, count, out);
    return hipGetLastError();
}

hipError_t launch_argmax_rows(const float* x, uint32_t rows, uint32_t width, uint32_t* out, uint64_t* partial,
                              uint32_t max_partials, int cus, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (width == 0) return hipErrorInvalidValue;
    // About 4 blocks per CU over all rows, at least 1024 columns (one trip) per
    // block, and no more keys than the partial buffer holds.
    uint64_t per_row = ((uint64_t)4 * (cus > 0 ? cus : 256) + rows - 1) / rows;
    const uint64_t trips = ((uint64_t)width + 1023) / 1024;
    if (per_row > trips) per_row = trips;
    if (per_row > max_partials / rows) per_row = max_partials / rows;
    if (per_row < 1) per_row = 1;
    uint32_t chunk = (uint32_t)(((uint64_t)width + per_row - 1) / per_row);
    if (chunk > (1u << 28)) return hipErrorInvalidValue;  // buffer-resource range of one piece
    const uint32_t chunks = (width + chunk - 1) / chunk;  // every piece starts below width
    const uint64_t grid = (uint64_t)rows * chunks;
    if (grid > 0x7fffffffu) return hipErrorInvalidValue;
    if (chunks == 1) {
        hipLaunchKernelGGL(argmax_chunk_kernel<true>, dim3((uint32_t)grid), dim3(256), 0, s, x, width, chunk, 1u,
                           partial, out);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(argmax_chunk_kernel<false>, dim3((uint32_t)grid), dim3(256), 0, s, x, width, chunk, chunks,
                       partial, out);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_argmax_reduce(partial, rows, chunks, out, s);
}

// ------------------------------------------------------------------ generator
//
// SplitMix64 output n of seed s; element i uses outputs 2i and 2i+1 as
// u1 in (0, 1] and u2 in [0, 1); z = sqrt(-2 ln u1) cos(2 pi u2) with the
// fixed polynomial ln and cos below (only +, -, *, /, sqrt, all correctly
// rounded and never contracted), then f32 = RNE(z * sigma), bf16 = RNE(f32).

__device__ __forceinline__ uint64_t splitmix64(uint64_t seed, uint64_t n) {
    uint64_t z = seed + (n + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ double synth_ln(double u) {
#pragma clang fp contract(off)
    const double inv_odd[13] = {
        0x1.0000000000000p+0, 0x1.5555555555555p-2, 0x1.999999999999ap-3,
        0x1.2492492492492p-3, 0x1.c71c71c71c71cp-4, 0x1.745d1745d1746p-4,
        0x1.3b13b13b13b14p-4, 0x1.1111111111111p-4, 0x1.e1e1e1e1e1e1ep-5,
        0x1.af286bca1af28p-5, 0x1.8618618618618p-5, 0x1.642c8590b2164p-5,
        0x1.47ae147ae147bp-5};
    uint64_t bits = __double_as_longlong(u);
    int e = (int)((bits >> 52) & 0x7ff) - 1023;
    bits = (bits & 0x000fffffffffffffull) | 0x3ff0000000000000ull;
    double m = __longlong_as_double(bits);
    if (m > 0x1.6a09e667f3bcdp+0) {
        m = m * 0.5;
        e += 1;
    }
    double t = (m - 1.0) / (m + 1.0);
    double t2 = t * t;
    double p = inv_odd[12];
#pragma unroll
    for (int k = 11; k >= 0; --k) p = p * t2 + inv_odd[k];
    return (double)e * 0x1.62e42fefa39efp-1 + 2.0 * t * p;
}

__device__ double synth_cos2pi(double turns) {
#pragma clang fp contract(off)
    const double inv_even_fact[17] = {
        0x1.0000000000000p+0, 0x1.0000000000000p-1, 0x1.5555555555555p-5,
        0x1.6c16c16c16c17p-10, 0x1.a01a01a01a01ap-16, 0x1.27e4fb7789f5cp-22,
        0x1.1eed8eff8d898p-29, 0x1.93974a8c07c9dp-37, 0x1.ae7f3e733b81fp-45,
        0x1.6827863b97d97p-53, 0x1.e542ba4020225p-62, 0x1.0ce396db7f853p-70,
        0x1.f2cf01972f578p-80, 0x1.88e85fc6a4e5ap-89, 0x1.0a18a2635085dp-98,
        0x1.3932c5047d60ep-108, 0x1.434d2e783f5bcp-118};
    double r = turns >= 0.5 ? turns - 1.0 : turns;
    double th = r * 0x1.921fb54442d18p+2;
    double th2 = th * th;
    double c = inv_even_fact[16];
#pragma unroll
    for (int k = 15; k >= 0; --k) {
        double a = (k & 1) ? -inv_even_fact[k] : inv_even_fact[k];
        c = a + th2 * c;
    }
    return c;
}

__device__ float synth_value(uint64_t seed, double sigma, uint64_t index) {
#pragma clang fp contract(off)
    uint64_t a = splitmix64(seed, 2 * index);
    uint64_t b = splitmix64(seed, 2 * index + 1);
    double u1 = (double)((a >> 11) + 1) * 0x1p-53;
    double u2 = (double)(b >> 11) * 0x1p-53;
    double z = __builtin_sqrt(-2.0 * synth_ln(u1)) * synth_cos2pi(u2);
    double zs = z * sigma;
    return (float)zs;
}

__global__ __launch_bounds__(256) void synth_bf16_kernel(uint64_t seed, double sigma, uint64_t start,
                                                         uint64_t count, uint16_t* __restrict__ out) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    out[i] = (uint16_t)f32_to_bf16_bits(synth_value(seed, sigma, start + i));
}

hipError_t launch_synth_bf16(uint64_t seed, double sigma, uint64_t start, uint64_t count, uint16_t* out,
                             hipStream_t s) {
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(synth_bf16_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, seed,
                       sigma, start, count, out);
    return hipGetLastError();
}

// Generate one 32-element block of bf16 values and quantize it in place:
// the weight recipe (bf16 N(0, sigma) from seed, MXFP4 by the reference rule)
// without materialising the bf16 tensor.
__global__ __launch_bounds__(256) void synth_weight_kernel(uint64_t seed, double sigma, uint64_t blocks,
                                                           uint8_t* __restrict__ packed,
                                                           uint8_t* __restrict__ scales) {
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    float v[32];
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        float f = synth_value(seed, sigma, b * 32 + i);
        v[i] = bf16_bits_to_f32(f32_to_bf16_bits(f));
        float a = __builtin_fabsf(v[i]);
        amax = a > amax ? a : amax;
    }
    const uint32_t s = mxfp4_scale_byte(amax);
    u32x4 out;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) word |= mxfp4_code(v[8 * d + i], s) << (4 * i);
        out[d] = word;
    }
    *reinterpret_cast<u32x4*>(packed + b * 16) = out;
    scales[b] = (uint8_t)s;
}

hipError_t launch_synth_weight(uint64_t seed, double sigma, uint32_t rows, uint32_t cols, uint8_t* packed,
                               uint8_t* scales, hipStream_t s) {
    const uint64_t blocks = (uint64_t)rows * (cols / 32);
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(synth_weight_kernel, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, s, seed,
                       sigma, blocks, packed, scales);
    return hipGetLastError();
}

}  // namespace mx4

namespace mx4 {

// A fill kernel instead of hipMemsetAsync, so callers may capture the
// enqueued work in a HIP graph.
__global__ void fill_u32_kernel(uint32_t* p, uint32_t count, uint32_t value) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = value;
}

hipError_t launch_fill_u32(uint32_t* p, uint32_t count, uint32_t value, hipStream_t s) {
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_u32_kernel, dim3((count + 255) / 256), dim3(256), 0, s, p, count, value);
    return hipGetLastError();
}

}  // namespace mx4
