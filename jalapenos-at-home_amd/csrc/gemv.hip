// gemv.hip -- exact MXFP4 x activation kernels for decode (M = 1) and the
// generic exact fallback (any M, any K % 32 == 0).
//
// Computes y[m, r] = sum_k x[m, k] * w(r, k), the product of
// engine/src/lib.rs:240-266, with w decoded from packed E2M1 + E8M0 per 32
// (engine/src/mxfp4.rs:27-33). Like the reference's fastest Metal kernel
// (project_token_blocks, engine/src/gpu.metal:324-356) the E8M0 scale is
// factored out of each 32-element block: the block's 32 products are summed
// with exact E2M1 levels, then multiplied once by 2^(s-127).
//
// gemv_m1 design (gfx950, HBM-bound):
//  * a team of WG waves owns R weight rows at a time; its 64*WG lanes split
//    each row's K/32 blocks, lane t taking blocks t + 64*WG*j (j < BPL), so
//    every 128-bit load instruction reads 1 KiB of contiguous packed bytes;
//  * the lane's activations for its BPL blocks are loaded once into VGPRs and
//    reused for every row the persistent team visits;
//  * the next row-set's loads are issued before the current one is reduced
//    (register double-buffering), keeping R*BPL KiB in flight per wave;
//  * E2M1 -> bf16/f32 by the hardware converter, bf16 dot2 (or f32 FMA)
//    accumulation, wave reduction through lane shuffles, cross-wave through LDS.
#include "mx4_device.h"
#include "mx4_kernels.h"

namespace mx4 {

template <bool XBF16, int BPL>
struct LaneX;

template <int BPL>
struct LaneX<true, BPL> {
    uint32_t p[BPL][16];  // bf16 pairs, element order
    __device__ __forceinline__ void load(const void* xv, uint32_t blk0, uint32_t stride) {
        const uint8_t* x = static_cast<const uint8_t*>(xv);
#pragma unroll
        for (int j = 0; j < BPL; ++j) {
            const uint8_t* src = x + (size_t)(blk0 + j * stride) * 64;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                u32x4 v = load_u32x4(src + 16 * q);
                p[j][4 * q + 0] = v[0];
                p[j][4 * q + 1] = v[1];
                p[j][4 * q + 2] = v[2];
                p[j][4 * q + 3] = v[3];
            }
        }
    }
    __device__ __forceinline__ float dot(int j, const u32x4 w) const { return block_dot_bf16(w, p[j]); }
};

template <int BPL>
struct LaneX<false, BPL> {
    float f[BPL][32];
    __device__ __forceinline__ void load(const void* xv, uint32_t blk0, uint32_t stride) {
        const float* x = static_cast<const float*>(xv);
#pragma unroll
        for (int j = 0; j < BPL; ++j) {
            const float* src = x + (size_t)(blk0 + j * stride) * 32;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                f32x4 v = *reinterpret_cast<const f32x4*>(src + 4 * q);
                f[j][4 * q + 0] = v[0];
                f[j][4 * q + 1] = v[1];
                f[j][4 * q + 2] = v[2];
                f[j][4 * q + 3] = v[3];
            }
        }
    }
    __device__ __forceinline__ float dot(int j, const u32x4 w) const { return block_dot_f32(w, f[j]); }
};

template <bool XBF16, int WG, int BPL, int R>
__global__ __launch_bounds__(64 * WG) void gemv_m1_kernel(const uint8_t* __restrict__ packed,
                                                          const uint8_t* __restrict__ scales,
                                                          const void* __restrict__ x,
                                                          float* __restrict__ y, uint32_t n,
                                                          uint32_t k, uint32_t rowsets) {
    constexpr uint32_t T = 64 * WG;
    const uint32_t t = threadIdx.x;
    const uint32_t wave = t / 64, lane = t % 64;
    const size_t row_bytes = k / 2;
    const uint32_t nblk = k / 32;

    LaneX<XBF16, BPL> xr;
    xr.load(x, t, T);

    __shared__ float red[2][WG][R];

    u32x4 wa[R][BPL];
    uint32_t sa[R][BPL];
    auto load_set = [&](uint32_t rs, u32x4 (&w)[R][BPL], uint32_t (&s)[R][BPL]) {
#pragma unroll
        for (int i = 0; i < R; ++i) {
            uint32_t row = rs * R + i;
            row = row < n ? row : n - 1;  // clamp: tail rows read a valid row, never written
            const uint8_t* prow = packed + row * row_bytes;
            const uint8_t* srow = scales + (size_t)row * nblk;
#pragma unroll
            for (int j = 0; j < BPL; ++j) {
                uint32_t b = t + j * T;
                w[i][j] = load_u32x4_nt(prow + 16 * (size_t)b);
                s[i][j] = srow[b];
            }
        }
    };

    uint32_t rs = blockIdx.x;
    if (rs >= rowsets) return;
    load_set(rs, wa, sa);
    uint32_t parity = 0;
    for (; rs < rowsets; rs += gridDim.x) {
        u32x4 wb[R][BPL];
        uint32_t sb[R][BPL];
        const uint32_t nxt = rs + gridDim.x;
        if (nxt < rowsets) load_set(nxt, wb, sb);

        float acc[R];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            float a = 0.0f;
#pragma unroll
            for (int j = 0; j < BPL; ++j) a = __builtin_fmaf(xr.dot(j, wa[i][j]), e8m0_to_f32(sa[i][j]), a);
            acc[i] = wave_sum(a);
        }
        if constexpr (WG == 1) {
            if (lane == 0) {
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    uint32_t row = rs * R + i;
                    if (row < n) y[row] = acc[i];
                }
            }
        } else {
            if (lane == 0) {
#pragma unroll
                for (int i = 0; i < R; ++i) red[parity][wave][i] = acc[i];
            }
            __syncthreads();
            if (t < R) {
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < WG; ++w) v += red[parity][w][t];
                uint32_t row = rs * R + t;
                if (row < n) y[row] = v;
            }
            parity ^= 1;
        }
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int j = 0; j < BPL; ++j) {
                wa[i][j] = wb[i][j];
                sa[i][j] = sb[i][j];
            }
    }
}

// Generic exact kernel: any M (tokens processed MT at a time), any K % 32 == 0.
// One wave per row; lanes stride over the row's blocks; activations are read
// from global memory (L1/L2-resident) for every block.
template <bool XBF16, int MT>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const uint8_t* __restrict__ packed,
                                                           const uint8_t* __restrict__ scales,
                                                           const void* __restrict__ xv,
                                                           float* __restrict__ y, uint32_t m,
                                                           uint32_t n, uint32_t k) {
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t row = blockIdx.x * 4 + threadIdx.x / 64;
    const uint32_t m0 = blockIdx.y * MT;
    if (row >= n) return;
    const uint32_t nblk = k / 32;
    const uint8_t* prow = packed + (size_t)row * (k / 2);
    const uint8_t* srow = scales + (size_t)row * nblk;
    float acc[MT];
#pragma unroll
    for (int q = 0; q < MT; ++q) acc[q] = 0.0f;
    for (uint32_t b = lane; b < nblk; b += 64) {
        u32x4 w = load_u32x4(prow + 16 * (size_t)b);
        float sc = e8m0_to_f32(srow[b]);
#pragma unroll
        for (int q = 0; q < MT; ++q) {
            uint32_t tok = m0 + q < m ? m0 + q : m - 1;
            float part;
            if constexpr (XBF16) {
                const uint8_t* src = static_cast<const uint8_t*>(xv) + ((size_t)tok * k + (size_t)b * 32) * 2;
                uint32_t xp[16];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    u32x4 v = load_u32x4(src + 16 * c);
                    xp[4 * c + 0] = v[0];
                    xp[4 * c + 1] = v[1];
                    xp[4 * c + 2] = v[2];
                    xp[4 * c + 3] = v[3];
                }
                part = block_dot_bf16(w, xp);
            } else {
                const float* src = static_cast<const float*>(xv) + (size_t)tok * k + (size_t)b * 32;
                float xf[32];
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    f32x4 v = *reinterpret_cast<const f32x4*>(src + 4 * c);
                    xf[4 * c + 0] = v[0];
                    xf[4 * c + 1] = v[1];
                    xf[4 * c + 2] = v[2];
                    xf[4 * c + 3] = v[3];
                }
                part = block_dot_f32(w, xf);
            }
            acc[q] = __builtin_fmaf(part, sc, acc[q]);
        }
    }
#pragma unroll
    for (int q = 0; q < MT; ++q) {
        float v = wave_sum(acc[q]);
        if (lane == 0 && m0 + q < m) y[(size_t)(m0 + q) * n + row] = v;
    }
}

// ------------------------------------------------------------------ launchers

struct M1Config {
    int wg, bpl, r;
};

template <bool XBF16, int WG, int BPL, int R>
static hipError_t launch_m1(const GemvArgs& a, int max_groups) {
    uint32_t rowsets = (a.n + R - 1) / R;
    uint32_t grid = rowsets < (uint32_t)max_groups ? rowsets : (uint32_t)max_groups;
    // even split: every team visits the same number of row-sets (+-1)
    uint32_t per = (rowsets + grid - 1) / grid;
    grid = (rowsets + per - 1) / per;
    hipLaunchKernelGGL((gemv_m1_kernel<XBF16, WG, BPL, R>), dim3(grid), dim3(64 * WG), 0, a.stream,
                       a.packed, a.scales, a.x, a.y, a.n, a.k, rowsets);
    return hipGetLastError();
}

template <bool XBF16>
static hipError_t dispatch_m1(const GemvArgs& a, int cus) {
    const uint32_t nblk = a.k / 32;
    // Waves per CU the persistent grid aims for; each wave keeps R*BPL KiB of
    // packed weights (plus the prefetched set) in flight.
    const int waves_per_cu = 8;
    switch (nblk) {
        case 64:  return launch_m1<XBF16, 1, 1, 4>(a, cus * waves_per_cu);
        case 128: return launch_m1<XBF16, 1, 2, 4>(a, cus * waves_per_cu);
        case 192: return launch_m1<XBF16, 1, 3, 2>(a, cus * waves_per_cu);
        case 256: return launch_m1<XBF16, 2, 2, 4>(a, cus * waves_per_cu / 2);
        case 384: return launch_m1<XBF16, 3, 2, 4>(a, cus * waves_per_cu / 3);
        default:  return hipErrorNotSupported;
    }
}

bool gemv_m1_supported(uint32_t k) {
    const uint32_t nblk = k / 32;
    return k % 32 == 0 && (nblk == 64 || nblk == 128 || nblk == 192 || nblk == 256 || nblk == 384);
}

hipError_t launch_gemv_m1(const GemvArgs& a, int cus) {
    return a.x_bf16 ? dispatch_m1<true>(a, cus) : dispatch_m1<false>(a, cus);
}

template <bool XBF16, int MT>
static hipError_t launch_generic_t(const GemvArgs& a) {
    dim3 grid((a.n + 3) / 4, (a.m + MT - 1) / MT);
    hipLaunchKernelGGL((gemv_generic_kernel<XBF16, MT>), grid, dim3(256), 0, a.stream, a.packed, a.scales,
                       a.x, a.y, a.m, a.n, a.k);
    return hipGetLastError();
}

hipError_t launch_gemv_generic(const GemvArgs& a) {
    if (a.m == 1) return a.x_bf16 ? launch_generic_t<true, 1>(a) : launch_generic_t<false, 1>(a);
    return a.x_bf16 ? launch_generic_t<true, 4>(a) : launch_generic_t<false, 4>(a);
}

}  // namespace mx4
