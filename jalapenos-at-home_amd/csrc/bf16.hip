// bf16.hip -- projections with bf16 (non-quantized) weights, the other arm of
// the reference's matmul: engine/src/lib.rs:240-266 with Tensor::bf16 weights
// (the `None` arm of lib.rs:255), which the Metal bridge takes when `scales`
// is NULL (engine/src/metal.rs:45-50, engine/src/metal.m:85-95).
//
// y[m, r] = sum_k x[m, k] * bf16_to_f32(w[r, k]), f32 accumulation. bf16 -> f32
// is exact (the top half of an f32), so the only difference from the
// reference's sequential loop is the summation order.
//
// One wave per weight row, MT tokens per wave: each lane streams 16-byte
// pieces (8 weights) of the row, fully coalesced, and reuses each piece for the
// MT activation rows; the wave then reduces with lane shuffles. Rows whose
// width is not a multiple of 8 (or is misaligned) take the element-wise form.
#include "mx4_device.h"
#include "mx4_kernels.h"

namespace mx4 {

namespace {

template <bool XBF16>
__device__ __forceinline__ void load_x8(const void* x, uint64_t elem, float (&v)[8]) {
    if constexpr (XBF16) {
        const u32x4 p = load_u32x4(static_cast<const uint8_t*>(x) + 2 * elem);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            v[2 * d] = bf16_bits_to_f32(p[d] & 0xffffu);
            v[2 * d + 1] = bf16_bits_to_f32(p[d] >> 16);
        }
    } else {
        const float* f = static_cast<const float*>(x) + elem;
        const f32x4 a = *reinterpret_cast<const f32x4*>(f);
        const f32x4 b = *reinterpret_cast<const f32x4*>(f + 4);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            v[d] = a[d];
            v[4 + d] = b[d];
        }
    }
}

template <bool XBF16>
__device__ __forceinline__ float load_x1(const void* x, uint64_t elem) {
    if constexpr (XBF16)
        return bf16_bits_to_f32(static_cast<const uint16_t*>(x)[elem]);
    else
        return static_cast<const float*>(x)[elem];
}

template <bool XBF16, int MT, bool VEC>
__global__ __launch_bounds__(256) void bf16_matmul_kernel(const uint16_t* __restrict__ w, const void* __restrict__ x,
                                                          float* __restrict__ y, uint32_t m, uint32_t n, uint32_t k) {
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t row = blockIdx.x * 4 + threadIdx.x / 64;
    const uint32_t m0 = blockIdx.y * MT;
    if (row >= n) return;
    const uint16_t* wr = w + (uint64_t)row * k;
    float acc[MT];
#pragma unroll
    for (int q = 0; q < MT; ++q) acc[q] = 0.0f;
    if constexpr (VEC) {
        for (uint32_t c = lane; c < k / 8; c += 64) {
            const u32x4 p = load_u32x4(reinterpret_cast<const uint8_t*>(wr) + 16 * (uint64_t)c);
            float wv[8];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                wv[2 * d] = bf16_bits_to_f32(p[d] & 0xffffu);
                wv[2 * d + 1] = bf16_bits_to_f32(p[d] >> 16);
            }
#pragma unroll
            for (int q = 0; q < MT; ++q) {
                const uint32_t tok = m0 + q < m ? m0 + q : m - 1;
                float xv[8];
                load_x8<XBF16>(x, (uint64_t)tok * k + 8 * (uint64_t)c, xv);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[q] = __builtin_fmaf(xv[e], wv[e], acc[q]);
            }
        }
    } else {
        for (uint32_t e = lane; e < k; e += 64) {
            const float wv = bf16_bits_to_f32(wr[e]);
#pragma unroll
            for (int q = 0; q < MT; ++q) {
                const uint32_t tok = m0 + q < m ? m0 + q : m - 1;
                acc[q] = __builtin_fmaf(load_x1<XBF16>(x, (uint64_t)tok * k + e), wv, acc[q]);
            }
        }
    }
#pragma unroll
    for (int q = 0; q < MT; ++q) {
        const float v = wave_sum(acc[q]);
        if (lane == 0 && m0 + q < m) y[(uint64_t)(m0 + q) * n + row] = v;
    }
}

template <bool XBF16, int MT>
hipError_t go(const uint16_t* w, const void* x, float* y, uint32_t m, uint32_t n, uint32_t k, bool vec,
              hipStream_t s) {
    dim3 grid((n + 3) / 4, (m + MT - 1) / MT);
    if (vec)
        hipLaunchKernelGGL((bf16_matmul_kernel<XBF16, MT, true>), grid, dim3(256), 0, s, w, x, y, m, n, k);
    else
        hipLaunchKernelGGL((bf16_matmul_kernel<XBF16, MT, false>), grid, dim3(256), 0, s, w, x, y, m, n, k);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_bf16_matmul(const uint16_t* w, const void* x, bool x_bf16, float* y, uint32_t m, uint32_t n,
                              uint32_t k, hipStream_t s) {
    if (m == 0 || n == 0 || k == 0) return hipSuccess;
    // 16-byte pieces need every row (weights and activations) to start 16-byte aligned
    const uint32_t xalign = x_bf16 ? 8 : 4;
    const bool vec = k % 8 == 0 && k % xalign == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0;
    if (m == 1) return x_bf16 ? go<true, 1>(w, x, y, m, n, k, vec, s) : go<false, 1>(w, x, y, m, n, k, vec, s);
    return x_bf16 ? go<true, 4>(w, x, y, m, n, k, vec, s) : go<false, 4>(w, x, y, m, n, k, vec, s);
}

}  // namespace mx4
